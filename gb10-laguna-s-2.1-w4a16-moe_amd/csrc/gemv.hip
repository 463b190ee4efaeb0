// Grouped dequant-GEMV launches for few tokens per expert: the GEMV-only
// kernel (its work item is in gemv_item.hpp) and the w2 + combine kernel of
// few-token calls.
#include <type_traits>

#include "common.hpp"
#include "gemv_item.hpp"

namespace w4a16 {
namespace {

using namespace gemv_dev;

#ifndef GEMV_MIN_WAVES
#define GEMV_MIN_WAVES 1
#endif

template <int MODE, int RPL, int PF, int TC, int WAVES, int NIT, bool ROUTE, int UPW, int LPR>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(GEMV_MIN_WAVES)))
void gemv_kernel(const GemvLaunch a) {
  extern __shared__ u32x4_t lds[];
  gemv_item<MODE, RPL, PF, TC, WAVES, NIT, ROUTE, UPW, LPR>(a, (int)blockIdx.x, lds);
}

// The w2 GEMV and the top-k combine of a few-token call in one launch.
//
// A workgroup has one wave per slot (topk <= 16) and owns 8 R output rows of
// one token (blockIdx.y); an expert routed from several tokens is read once
// per token.
// Wave t computes slot t's 8 R rows exactly as gemv_kernel<1, ...> does (8
// lanes per row on groups 8*it + lane%8, the same dot2 chain per word and
// fma per group, the same 8-lane sum), multiplies by the routing weight and
// parks the value in LDS.  The workgroup then adds the slots in order from
// 0.0, skipping ids outside [0, E), as combine_kernel does.  The result is
// therefore bit-identical to gemv_kernel + combine_kernel (with the same
// bf16 rounding of each weighted slot value when the call keeps bf16 partial
// rows), with one launch, no partial rows in memory, and every wave's weight
// loads in flight at once.
template <int NIT, int R>
__global__ __launch_bounds__(1024) void w2_token_kernel(const GemvLaunch a, uint16_t* out,
                                                       int64_t ld_out) {
  extern __shared__ u32x4_t lds[];
  const int topk = a.topk;
  const int t = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // this wave's slot
  const int m = blockIdx.y;                                          // token
  const int f = m * topk + t;                                        // flat slot
  const int lane = __lane_id();
  const int kdim = a.kdim;
  const int G = kdim >> 5;
  const int gpr = kdim / a.group;
  const int gshift = a.group == 32 ? 0 : (a.group == 64 ? 1 : 2);
  const int row_oct = staged_row_octets(kdim);
  u32x4_t* xp = lds + t * row_oct;
  float* xc = reinterpret_cast<float*>(lds + topk * row_oct) + t * (G + 1);
  float* red = reinterpret_cast<float*>(lds + topk * row_oct) + topk * (G + 1);  // [topk][8R]

  const int E = a.num_experts;
  const int e_raw = a.ids[f];
  const float wt = a.topk_w[f];  // loaded with the id, used at the end
  const bool valid = e_raw >= 0 && e_raw < E;  // wave-uniform
  const int e = valid ? e_raw : 0;
  // The slot's intermediate row: with the step count fixed at compile time
  // its pieces are loaded together (one round trip instead of one per piece)
  // and staged before the weight loads are issued.
  if constexpr (NIT > 0) {
    constexpr int kStageIt = (NIT * 32 + 4 + 63) / 64;  // row octets + zero group
    const int n_oct = kdim >> 3;
    const u32x4_t* xrow = reinterpret_cast<const u32x4_t*>(a.act + (int64_t)f * a.ld_act);
    u32x4_t xs[kStageIt];
#pragma unroll
    for (int i = 0; i < kStageIt; ++i) {
      const int u = i * 64 + lane;
      xs[i] = u32x4_t{0u, 0u, 0u, 0u};
      if (u < n_oct) xs[i] = xrow[u];
    }
#pragma unroll
    for (int i = 0; i < kStageIt; ++i)
      if (i * 64 < n_oct + 4) stage_octet(xs[i], i * 64 + lane, n_oct, xp, xc, lane);
  } else {
    stage_row<64>(a.act + (int64_t)f * a.ld_act, kdim, xp, xc, lane);
  }

  // Lane (r, sl) owns rows rb0 + r + 8 j, j < R, of the workgroup's 8 R.
  const int r = lane >> 3, sl = lane & 7;
  const int rb0 = blockIdx.x * 8 * R;
  const char* wrow = reinterpret_cast<const char*>(a.w) + ((int64_t)e * a.n_out + rb0 + r) * G * 16;
  const char* srow = reinterpret_cast<const char*>(a.s) + ((int64_t)e * a.n_out + rb0 + r) * gpr * 2;
  const int64_t wstep = (int64_t)8 * G * 16, sstep = (int64_t)8 * gpr * 2;  // 8 rows on
  const uint32_t mask = a.nib_mask;
  uint32_t magic;
  asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "s"(a.nib_magic));
  const int n_it = NIT > 0 ? NIT : (G + 7) >> 3;
  constexpr int kMaxIt = NIT > 0 ? NIT : 1;

  // All loads first (NIT x R of them), then the staged row is ready.
  u32x4_t wq[R][kMaxIt];
  uint32_t sq[R][kMaxIt];
  if constexpr (NIT > 0) {
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int gi = min(it * 8 + sl, G - 1);
        wq[j][it] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t*>(wrow + j * wstep + gi * 16));
        sq[j][it] = *reinterpret_cast<const uint16_t*>(srow + j * sstep + (gi >> gshift) * 2);
      }
  }
  __syncthreads();

  auto step = [&](const u32x4_t& w4, uint32_t sbits, int it, float& acc) {
    const int gi = it * 8 + sl;
    const int gl = gi < G ? gi : G;
    float pj = xc[gl];  // -C
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const u32x4_t x = xp[lds_octet(gl * 4 + w)];
      const uint32_t wv = w4[w];
      const uint32_t d0 = (wv & mask) | magic;
      const uint32_t d1 = ((wv >> 4) & mask) | magic;
      const uint32_t d2 = ((wv >> 8) & mask) | magic;
      const uint32_t d3 = ((wv >> 12) & mask) | magic;
      float q = dot2(d0, x[0], pj);
      q = dot2(d1, x[1], q);
      q = dot2(d2, x[2], q);
      pj = dot2(d3, x[3], q);
    }
    acc = fmaf(bf16_to_f32(sbits), pj, acc);
  };
#pragma unroll
  for (int j = 0; j < R; ++j) {
    float acc = 0.0f;
    if constexpr (NIT > 0) {
#pragma unroll
      for (int it = 0; it < NIT; ++it) step(wq[j][it], sq[j][it], it, acc);
    } else {
      for (int it = 0; it < n_it; ++it) {
        const int gi = min(it * 8 + sl, G - 1);
        const u32x4_t w4 = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t*>(wrow + j * wstep + gi * 16));
        const uint32_t sb =
            *reinterpret_cast<const uint16_t*>(srow + j * sstep + (gi >> gshift) * 2);
        step(w4, sb, it, acc);
      }
    }
    acc = oct_sum(acc);
    // The weighted slot value is rounded to bf16 when the call keeps bf16
    // partial rows (M > 4), as gemv_kernel<1> stores it for combine_kernel.
    float v = acc * wt;
    if (a.partial_bf16) v = bf16_to_f32(f32_to_bf16(v));
    // A slot routed outside [0, E) parks +0.0: the sum starts at +0.0 and so
    // is never -0.0, and adding +0.0 to any other value leaves it unchanged,
    // so summing every slot equals skipping those -- without reading the ids
    // again here.
    if (sl == 0) red[t * 8 * R + r + 8 * j] = valid ? v : 0.0f;
  }
  __syncthreads();
  if (threadIdx.x < 8 * R) {
    float sum = 0.0f;
    for (int s = 0; s < topk; ++s) sum += red[s * 8 * R + threadIdx.x];
    out[(int64_t)m * ld_out + rb0 + threadIdx.x] = (uint16_t)f32_to_bf16(sum);
  }
}

// Output rows per workgroup of the one-launch w2 + top-k sum, in blocks of 8
// (each lane owns R rows): R = 2 from 3 tokens up, else 1.  Measured on
// MI355X (E=256, top-10, K=3072, N=1024): M=4 18.2 -> 16.9 us for the w2
// launch with R = 2; M=1 7.2 -> 7.6 us and M=2 11.3 -> 11.7 us, so those
// keep R = 1; R = 4 is slower at every M.
constexpr int kW2TokenRMax = 2;
constexpr int kW2TokenR2MinM = 3;
int pick_w2_token_r(int M, int K) {
  return (M >= kW2TokenR2MinM && K % (8 * kW2TokenRMax) == 0) ? kW2TokenRMax : 1;
}

size_t w2_token_lds_bytes(int topk, int kdim) {
  return (size_t)topk * (staged_row_octets(kdim) * sizeof(u32x4_t) +
                         (size_t)((kdim >> 5) + 1) * sizeof(float)) +
         (size_t)topk * 8 * kW2TokenRMax * sizeof(float);
}



// Fully unrolled step loops (NIT fixed at compile time) for the row lengths
// of the benchmark shape; 0 keeps the run-time loop.  Overridable at build
// time for tuning sweeps.
#ifndef W4A16_W13_UNROLL
#define W4A16_W13_UNROLL 1
#endif
#ifndef W4A16_W2_UNROLL
#define W4A16_W2_UNROLL 1
#endif

template <int MODE, int RPL, int PF, int TC, int NIT, bool ROUTE, int UPW, int LPR>
hipError_t launch_gemv_n(const GemvLaunch& a, hipStream_t stream) {
  constexpr int W = kGemvWaves;
  const int rows_per_wave = (64 / LPR) * RPL;
  if (a.n_out % rows_per_wave != 0) return hipErrorInvalidValue;
  const int chunks = a.n_out / rows_per_wave;
  const int slabs = (chunks + W - 1) / W;
  const int groups = (slabs + UPW - 1) / UPW;
  const size_t lds =
      ROUTE ? gemv_route_lds_bytes(TC, a.kdim, a.num_experts) : gemv_lds_bytes(TC, a.kdim);
  if (lds > kMaxLds) return hipErrorInvalidValue;
  if (ROUTE && (a.n_tok < 1 || a.n_tok > kRouteMaxTok)) return hipErrorInvalidValue;
  const int64_t grid = (int64_t)(ROUTE ? a.max_items : a.max_blocks) * groups;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL((gemv_kernel<MODE, RPL, PF, TC, W, NIT, ROUTE, UPW, LPR>), dim3((unsigned)grid),
                     dim3(64 * W), lds, stream, a);
  return hipGetLastError();
}

// Units (row slabs) per workgroup: a.upw, else 1.  Measured on MI355X
// (E=256, top-10, M=4..64): more units per workgroup lose -- the w13 variant
// drops to two waves per SIMD, and under skewed routing an expert with many
// pairs becomes a few long workgroups (M=16 skewed: 184 vs 104 us per call).
template <int PF, int NIT>
int pick_upw(const GemvLaunch& a, int slabs) {
  (void)slabs;
  if (NIT == 0 || NIT % PF != 0) return 1;
  return a.upw > 0 ? a.upw : 1;
}

template <int MODE, int RPL, int PF, int TC, int NIT, bool ROUTE, int LPR>
hipError_t launch_gemv_u(const GemvLaunch& a, hipStream_t stream) {
  const int chunks = a.n_out / ((64 / LPR) * RPL);
  const int slabs = (chunks + kGemvWaves - 1) / kGemvWaves;
  if constexpr (LPR == 8 && NIT > 0 && NIT % PF == 0) {
    switch (pick_upw<PF, NIT>(a, slabs)) {
      case 4: return launch_gemv_n<MODE, RPL, PF, TC, NIT, ROUTE, 4, LPR>(a, stream);
      case 2: return launch_gemv_n<MODE, RPL, PF, TC, NIT, ROUTE, 2, LPR>(a, stream);
      default: break;
    }
  }
  return launch_gemv_n<MODE, RPL, PF, TC, NIT, ROUTE, 1, LPR>(a, stream);
}

// Fully unrolled step loops for the row lengths of the target layer
// (K = 3072: 12 steps; N = 1024: 4 steps); any other length runs the loop.
template <int MODE, int RPL, int PF, int TC, bool ROUTE, int LPR>
hipError_t launch_gemv_r(const GemvLaunch& a, hipStream_t stream) {
  const int n_it = ((a.kdim >> 5) + LPR - 1) / LPR;
  constexpr bool unroll = MODE == 0 ? W4A16_W13_UNROLL : W4A16_W2_UNROLL;
  if (!unroll) return launch_gemv_u<MODE, RPL, PF, TC, 0, ROUTE, LPR>(a, stream);
  if constexpr (LPR == 8) {
    switch (n_it) {
      case 4: return launch_gemv_u<MODE, RPL, PF, TC, 4, ROUTE, LPR>(a, stream);
      case 12: return launch_gemv_u<MODE, RPL, PF, TC, 12, ROUTE, LPR>(a, stream);
      default: break;
    }
  } else if constexpr (LPR == 32) {
    switch (n_it) {
      case 1: return launch_gemv_u<MODE, RPL, PF, TC, 1, ROUTE, LPR>(a, stream);
      case 3: return launch_gemv_u<MODE, RPL, PF, TC, 3, ROUTE, LPR>(a, stream);
      default: break;
    }
  }
  return launch_gemv_u<MODE, RPL, PF, TC, 0, ROUTE, LPR>(a, stream);
}

template <int MODE, int RPL, int PF, int TC, int LPR = 8>
hipError_t launch_gemv_t(const GemvLaunch& a, hipStream_t stream) {
  return a.ids ? launch_gemv_r<MODE, RPL, PF, TC, true, LPR>(a, stream)
               : launch_gemv_r<MODE, RPL, PF, TC, false, LPR>(a, stream);
}


}  // namespace



// R, P: rows per lane and steps in flight of passes of one or two token
// rows; R4, P4: those of four-row passes.
template <int MODE, int R, int P, int R4 = R, int P4 = P>
hipError_t launch_gemv_tc(const GemvLaunch& a, hipStream_t stream) {
  const int tc = pick_tc(a, a.num_experts);
  const bool wide = pick_lpr(a, tc, MODE) == 32;
  switch (tc) {
    case 1: return wide ? launch_gemv_t<MODE, R, P, 1, 32>(a, stream)
                        : launch_gemv_t<MODE, R, P, 1>(a, stream);
    case 2: return wide ? launch_gemv_t<MODE, R, P, 2, 32>(a, stream)
                        : launch_gemv_t<MODE, R, P, 2>(a, stream);
    default: return launch_gemv_t<MODE, R4, P4, 4>(a, stream);
  }
}

hipError_t launch_w13_gemv(const GemvLaunch& a_in, hipStream_t stream) {
  GemvLaunch a = a_in;
  a.nib_mask = 0x000F000Fu;
  a.nib_magic = 0x43004300u;  // bf16 (128, 128)
  return launch_gemv_tc<0, W4A16_W13_RPL, W4A16_W13_PF, W4A16_W13_RPL_T4, W4A16_W13_PF_T4>(a,
                                                                                       stream);
}

bool gemv_route_fits(int n_tok, int num_experts, int K, int N) {
  return n_tok >= 1 && n_tok <= kRouteMaxTok &&
         gemv_route_lds_bytes(1, K, num_experts) <= kMaxLds &&
         gemv_route_lds_bytes(1, N, num_experts) <= kMaxLds;
}

bool w2_token_fits(int topk, int K, int N) {
  return topk >= 1 && topk <= 16 && K % 8 == 0 && w2_token_lds_bytes(topk, N) <= kMaxLds;
}

hipError_t launch_w2_token(const GemvLaunch& a_in, uint16_t* out, int64_t ld_out,
                           hipStream_t stream) {
  GemvLaunch a = a_in;
  a.nib_mask = 0x000F000Fu;
  a.nib_magic = 0x43004300u;
  if (!w2_token_fits(a.topk, a.n_out, a.kdim)) return hipErrorInvalidValue;
  const int M = a.n_tok / a.topk;
  const int R = pick_w2_token_r(M, a.n_out);
  const dim3 grid((unsigned)(a.n_out / (8 * R)), (unsigned)M), block(64 * a.topk);
  const size_t lds = w2_token_lds_bytes(a.topk, a.kdim);
  const int n_it = ((a.kdim >> 5) + 7) >> 3;
  if (n_it == 4 && R == 2)
    hipLaunchKernelGGL((w2_token_kernel<4, 2>), grid, block, lds, stream, a, out, ld_out);
  else if (n_it == 4)
    hipLaunchKernelGGL((w2_token_kernel<4, 1>), grid, block, lds, stream, a, out, ld_out);
  else if (R == 2)
    hipLaunchKernelGGL((w2_token_kernel<0, 2>), grid, block, lds, stream, a, out, ld_out);
  else
    hipLaunchKernelGGL((w2_token_kernel<0, 1>), grid, block, lds, stream, a, out, ld_out);
  return hipGetLastError();
}

hipError_t launch_w2_gemv(const GemvLaunch& a_in, hipStream_t stream) {
  GemvLaunch a = a_in;
  a.nib_mask = 0x000F000Fu;
  a.nib_magic = 0x43004300u;
  return launch_gemv_tc<1, W4A16_W2_RPL, W4A16_W2_PF, W4A16_W2_RPL_T4, W4A16_W2_PF_T4>(a, stream);
}

}  // namespace w4a16
