// Grouped dequant-GEMM on bf16 MFMA for experts with many tokens (prefill).
//
// Reference kernels: _w4a16_moe_w1_fused_kernel (kernels/w4a16_moe.py:374-499)
// and _w4a16_moe_w2_kernel (:502-634): per 16-token block x 64-column tile,
// tl.dot of bf16 activations with bf16(dequantized weights), fp32 accumulate.
//
// Here one workgroup (4 waves) owns a tile of up to 128 sorted token slots of
// one expert x 256 weight rows and walks the reduction axis one 32-element
// group (one step) at a time:
//   * packed weights arrive in slabs of 8 groups: 8 lanes read one row's
//     128-byte line, so every load instruction covers whole lines; a slab is
//     fetched into registers one slab ahead and parked in LDS (packed, 136 B
//     per row) together with its scales converted to fp32;
//   * each wave owns 64 of the 256 weight rows and dequantizes exactly the
//     MFMA B fragments it needs straight from the packed slab: lane
//     (j = lane % 32, q = lane / 32) reads the two packed words 2q, 2q+1 of
//     its row's group and turns each into 8 bf16 values
//     bf16((code-8) * scale) -- exact in fp32 before the rounding, i.e. the
//     reference's dequantized weight;
//   * the gathered activation rows of one group go through a double-buffered
//     LDS tile (80 B per row), loaded two steps ahead;
//   * per group each wave issues 16 v_mfma_f32_32x32x16_bf16: 4 token blocks
//     of 32 x its 2 weight blocks of 32 x 2 halves of the group.  Half `sub`
//     contracts the k-octets 2q+sub of the group (A and B agree on it), so a
//     lane's two packed words feed both halves.
//
// w13 (MODE 0): wave w owns gate rows 32w.. and the matching up rows, so each
// lane holds gate and up of the same output column and the epilogue writes
// bf16(SiLU(gate) * up) -- the reference's rounding point.
// w2 (MODE 1): the epilogue multiplies by the routing weight and writes the
// fp32 partial row of the (token, slot) pair.
//
// Workgroup ids are remapped so that the N-tiles of one token tile run on one
// XCD (consecutive hardware ids round-robin over the 8 XCDs) and share its L2
// for the activation rows.
#include "common.hpp"

namespace w4a16 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// Native vectors: whole-value copies of HIP's union-based 4-vector structs
// end up in scratch memory instead of registers.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTM = kMfmaTileM;          // token slots per tile (4 blocks of 32)
constexpr int kTN = kMfmaTileN;          // weight rows per tile (8 blocks of 32)
constexpr int kSlab = 8;                 // groups per packed weight slab
constexpr int kApitch = 32 * 2 + 16;     // bytes per activation row in LDS
constexpr int kAbytes = kTM * kApitch;
constexpr int kBpitch = kSlab * 16 + 8;  // bytes per packed weight row in LDS
constexpr int kBbytes = kTN * kBpitch;
constexpr int kSpitch = kSlab + 1;       // fp32 scales per row in LDS
constexpr int kSbytes = kTN * kSpitch * 4;
constexpr int kLdsBytes = 2 * kAbytes + kBbytes + kSbytes;
constexpr int kXcds = 8;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// 8 codes of one packed word -> 8 bf16 (code - 8) * s in k order.
__device__ __forceinline__ bf16x8_t dequant_word(uint32_t w, float s) {
  const float b = -8.0f * s;
  const uint32_t lo = w & 0x0F0F0F0Fu;         // codes 0,2,4,6
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // codes 1,3,5,7
  const float v0 = fmaf((float)(lo & 0xFFu), s, b);
  const float v1 = fmaf((float)(hi & 0xFFu), s, b);
  const float v2 = fmaf((float)((lo >> 8) & 0xFFu), s, b);
  const float v3 = fmaf((float)((hi >> 8) & 0xFFu), s, b);
  const float v4 = fmaf((float)((lo >> 16) & 0xFFu), s, b);
  const float v5 = fmaf((float)((hi >> 16) & 0xFFu), s, b);
  const float v6 = fmaf((float)(lo >> 24), s, b);
  const float v7 = fmaf((float)(hi >> 24), s, b);
  const u32x4_t o = {pack_bf16x2(v0, v1), pack_bf16x2(v2, v3), pack_bf16x2(v4, v5),
                     pack_bf16x2(v6, v7)};
  return __builtin_bit_cast(bf16x8_t, o);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int per = n / kXcds;
  if (bid >= per * kXcds) return bid;
  return (bid % kXcds) * per + bid / kXcds;
}

// GSHIFT = log2(group / 32), a template parameter so that the scale loads
// are branch-free (branches around loads make the compiler wait for them).
template <int MODE, int GSHIFT>
__global__ __launch_bounds__(256, 2) void mfma_kernel(const MfmaLaunch a) {
  constexpr int gshift = GSHIFT;
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int s_f[kTM];
  unsigned char* const A0 = lds;
  unsigned char* const Bp = lds + 2 * kAbytes;
  float* const Sc = reinterpret_cast<float*>(Bp + kBbytes);

  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  const int n_tiles_n = rows_total / kTN;
  // The grid is sized for the most tiles a routing can produce; the align
  // kernel wrote the real count.  Workgroups past it leave at once, and the
  // XCD remap runs over the real ones so that every XCD gets its share.
  const int n_active = a.header[2] * n_tiles_n;
  if ((int)blockIdx.x >= n_active) return;
  const int bid = xcd_remap(blockIdx.x, n_active);
  const int tile = bid / n_tiles_n;
  const int nt = bid - tile * n_tiles_n;
  const int4 info = a.tiles[tile];
  const int e = info.x, start = info.y, count = info.z;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);

  for (int i = tid; i < kTM; i += 256) s_f[i] = i < count ? a.sorted[start + i] : a.n_tok;
  __syncthreads();

  const int kdim = a.kdim;
  const int G = kdim >> 5;  // steps; a multiple of kSlab on this path
  const int gpr = kdim / a.group;
  const int nslabs = G / kSlab;

  // ---- activation loads: two 16-byte octets per thread per step ----------
  // Rows past the tile's count read row 0 (their results are discarded).
  const u32x4_t* a_src[2];
  int a_lds[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int u = tid + 256 * i;
    const int row = u >> 2, part = u & 3;
    const int f = s_f[row];
    int64_t arow = 0;
    if (f < a.n_tok) arow = MODE == 0 ? f / a.topk : f;
    a_src[i] = reinterpret_cast<const u32x4_t*>(a.act + arow * a.ld_act) + part;
    a_lds[i] = row * kApitch + part * 16;
  }

  // ---- packed weight slabs: row (32i + tid/8), group tid%8, i = 0..7 ------
  auto global_row = [&](int r) {
    if (MODE == 0) {
      const int half = kTN / 2;
      return r < half ? nt * half + r : a.n_out + nt * half + (r - half);
    }
    return nt * kTN + r;
  };
  const int64_t e_rows = (int64_t)e * rows_total;
  const char* wexp = reinterpret_cast<const char*>(a.w) + e_rows * G * 16;
  const int bgrp = tid & 7;
  uint32_t b_off[kSlab];  // byte offset of this thread's 8 rows at group bgrp
#pragma unroll
  for (int i = 0; i < kSlab; ++i)
    b_off[i] = (uint32_t)global_row(32 * i + (tid >> 3)) * (uint32_t)G * 16u +
               (uint32_t)bgrp * 16u;
  // Scales of row tid: kSlab >> gshift bf16 values per slab.
  const char* s_row = reinterpret_cast<const char*>(a.s + (e_rows + global_row(tid)) * gpr);

  u32x4_t bs[kSlab];
  u32x4_t ss;
  auto load_slab = [&](int slab) {
    const int sl = min(slab, nslabs - 1);
    const uint32_t step_off = (uint32_t)sl * kSlab * 16u;
#pragma unroll
    for (int i = 0; i < kSlab; ++i)
      bs[i] = *reinterpret_cast<const u32x4_t*>(wexp + (b_off[i] + step_off));
    const char* sp = s_row + ((sl * kSlab) >> gshift) * 2;
    if constexpr (GSHIFT == 0) {
      ss = *reinterpret_cast<const u32x4_t*>(sp);
    } else if constexpr (GSHIFT == 1) {
      const u32x2_t v = *reinterpret_cast<const u32x2_t*>(sp);
      ss = u32x4_t{v[0], v[1], 0u, 0u};
    } else {
      ss = u32x4_t{*reinterpret_cast<const uint32_t*>(sp), 0u, 0u, 0u};
    }
  };
  auto store_slab = [&]() {
#pragma unroll
    for (int i = 0; i < kSlab; ++i) {
      unsigned char* d = Bp + (32 * i + (tid >> 3)) * kBpitch + bgrp * 16;
      *reinterpret_cast<u32x2_t*>(d) = u32x2_t{bs[i][0], bs[i][1]};
      *reinterpret_cast<u32x2_t*>(d + 8) = u32x2_t{bs[i][2], bs[i][3]};
    }
    float* srow = Sc + tid * kSpitch;
#pragma unroll
    for (int g = 0; g < kSlab; ++g) {
      const int si = g >> gshift;  // scale index within the slab
      const uint32_t word = ss[si >> 1];
      srow[g] = bf16_to_f32((si & 1) ? (word >> 16) : (word & 0xFFFFu));
    }
  };

  // ---- per-wave fragment geometry -----------------------------------------
  const int j = lane & 31;
  const int q = lane >> 5;
  int nrow[2];  // local weight row of this lane in each of the wave's 2 blocks
  if (MODE == 0) {
    nrow[0] = 32 * wid + j;             // gate
    nrow[1] = kTN / 2 + 32 * wid + j;   // matching up
  } else {
    nrow[0] = 64 * wid + j;
    nrow[1] = 64 * wid + 32 + j;
  }
  const int mcount = (count + 31) >> 5;  // active 32-token blocks (wave-uniform)

  f32x16_t acc[4][2];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.0f;

  struct AStage {
    u32x4_t v0, v1;
  };
  auto load_a = [&](AStage& st, int step) {
    const int k = min(step, G - 1);
    st.v0 = a_src[0][k * 4];
    st.v1 = a_src[1][k * 4];
  };

  // One reduction step (group g of the current slab).
  auto step_body = [&](AStage& st, unsigned char* Ab, int step, int g, bool slab_start,
                       int slab) {
    *reinterpret_cast<u32x4_t*>(Ab + a_lds[0]) = st.v0;
    *reinterpret_cast<u32x4_t*>(Ab + a_lds[1]) = st.v1;
    __syncthreads();
    if (slab_start) {
      // Every wave is past the previous slab's last reads: park this slab.
      store_slab();
      __syncthreads();
      load_slab(slab + 1);
    }
    load_a(st, step + 2);
    bf16x8_t bfr[2][2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const u32x2_t wv =
          *reinterpret_cast<const u32x2_t*>(Bp + nrow[n] * kBpitch + g * 16 + q * 8);
      const float sc = Sc[nrow[n] * kSpitch + g];
      bfr[n][0] = dequant_word(wv[0], sc);
      bfr[n][1] = dequant_word(wv[1], sc);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m < mcount) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(
              Ab + (m * 32 + j) * kApitch + (2 * q + sub) * 16);
#pragma unroll
          for (int n = 0; n < 2; ++n)
            acc[m][n] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bfr[n][sub], acc[m][n], 0, 0, 0);
        }
      }
    }
  };

  // Prologue in the order the loop expects (slab, then steps 0 and 1).
  AStage st0, st1;
  load_slab(0);
  __builtin_amdgcn_sched_barrier(0);
  load_a(st0, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_a(st1, 1);

  for (int slab = 0; slab < nslabs; ++slab) {
    const int s0 = slab * kSlab;
#pragma unroll
    for (int g = 0; g < kSlab; g += 2) {
      step_body(st0, A0, s0 + g, g, g == 0, slab);
      step_body(st1, A0 + kAbytes, s0 + g + 1, g + 1, false, slab);
    }
  }

  // Epilogue.  Accumulator register r of a 32x32 block holds row
  // 8*(r/4) + 4*(lane/32) + r%4 and column lane%32.
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if (m >= mcount) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int trow = m * 32 + 8 * (r >> 2) + 4 * q + (r & 3);
      const int f = s_f[trow];
      if (f >= a.n_tok) continue;
      if (MODE == 0) {
        uint16_t* out = static_cast<uint16_t*>(a.out) + (int64_t)f * a.n_out;
        const float h = silu(acc[m][0][r]) * acc[m][1][r];
        out[nt * (kTN / 2) + 32 * wid + j] = (uint16_t)f32_to_bf16(h);
      } else {
        const float wt = a.topk_w[f];
        float* out = static_cast<float*>(a.out) + (int64_t)f * a.n_out;
        out[nt * kTN + 64 * wid + j] = acc[m][0][r] * wt;
        out[nt * kTN + 64 * wid + 32 + j] = acc[m][1][r] * wt;
      }
    }
  }
}

template <int MODE>
hipError_t launch_mfma_t(const MfmaLaunch& a, hipStream_t stream) {
  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  if (rows_total % kTN != 0 || a.kdim % (32 * kSlab) != 0) return hipErrorInvalidValue;
  const int64_t grid = (int64_t)a.max_tiles * (rows_total / kTN);
  if (grid <= 0) return hipSuccess;
  const dim3 g((unsigned)grid), b(256);
  switch (a.group) {
    case 32: hipLaunchKernelGGL((mfma_kernel<MODE, 0>), g, b, kLdsBytes, stream, a); break;
    case 64: hipLaunchKernelGGL((mfma_kernel<MODE, 1>), g, b, kLdsBytes, stream, a); break;
    case 128: hipLaunchKernelGGL((mfma_kernel<MODE, 2>), g, b, kLdsBytes, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_w13_mfma(const MfmaLaunch& a, hipStream_t stream) {
  return launch_mfma_t<0>(a, stream);
}

hipError_t launch_w2_mfma(const MfmaLaunch& a, hipStream_t stream) {
  return launch_mfma_t<1>(a, stream);
}

}  // namespace w4a16
