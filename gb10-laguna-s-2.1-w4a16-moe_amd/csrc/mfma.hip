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
// partial row of the (token, slot) pair, rounded to bf16 like the
// reference's partial buffer (kernels/w4a16_moe.py:311) unless the call
// keeps fp32 partials (M <= 4, where the reference accumulates in fp32).
//
// Workgroup ids are remapped so that the N-tiles of one token tile run on one
// XCD (consecutive hardware ids round-robin over the 8 XCDs) and share its L2
// for the activation rows.
#include <type_traits>

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

constexpr int kTN = kMfmaTileN;          // weight rows per tile (8 blocks of 32)
constexpr int kSlab = 4;                 // groups per packed weight slab
constexpr int kApitch = 32 * 2 + 16;     // bytes per activation row in LDS
constexpr int kBpitch = kSlab * 16 + 8;  // bytes per packed weight row in LDS
constexpr int kBbytes = kTN * kBpitch;
constexpr int kSpitch = kSlab + 1;       // fp32 scales per row in LDS
constexpr int kSbytes = kTN * kSpitch * 4;
constexpr int kXcds = 8;

// Token tile of TMB blocks of 32 slots.
template <int TMB>
constexpr int lds_bytes() {
  return 2 * (32 * TMB) * kApitch + kBbytes + kSbytes;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// 8 codes of one packed word -> 8 bf16 (code - 8) * s in k order.  The
// masked nibble registers are made opaque so that the byte conversions read
// them directly (v_cvt_f32_ubyte0..3) instead of re-extracting each nibble.
__device__ __forceinline__ bf16x8_t dequant_word(uint32_t w, float s, float b) {
  uint32_t lo = w & 0x0F0F0F0Fu;         // codes 0,2,4,6
  uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // codes 1,3,5,7
  asm volatile("" : "+v"(lo), "+v"(hi));
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
// TMB = token blocks of 32 per tile: 4 (two workgroups per CU) or 8 (one;
// for large batches, where a 256-slot tile holds a whole expert and its
// weights are dequantized once instead of once per 128 tokens).
template <int MODE, int GSHIFT, int TMB>
__global__ __launch_bounds__(256, TMB == 8 ? 1 : 2) void mfma_kernel(const MfmaLaunch a) {
  constexpr int gshift = GSHIFT;
  constexpr int kTM = 32 * TMB;
  constexpr int kAbytes = kTM * kApitch;
  constexpr int NA = kTM * 4 / 256;  // activation octets per thread per step
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

  // ---- activation loads: NA 16-byte octets per thread per step -----------
  // Rows past the tile's count read row 0 (their results are discarded).
  const u32x4_t* a_src[NA];
  int a_lds[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int u = tid + 256 * i;
    const int row = u >> 2, part = u & 3;
    const int f = s_f[row];
    int64_t arow = 0;
    if (f < a.n_tok) arow = MODE == 0 ? f / a.topk : f;
    a_src[i] = reinterpret_cast<const u32x4_t*>(a.act + arow * a.ld_act) + part;
    a_lds[i] = row * kApitch + part * 16;
  }

  // ---- packed weight slabs: kSlab lanes per row (one group each), rows
  // (256 / kSlab) * i + tid / kSlab for i < kSlab -------------------------
  constexpr int kRowsPerPass = 256 / kSlab;
  auto global_row = [&](int r) {
    if (MODE == 0) {
      const int half = kTN / 2;
      return r < half ? nt * half + r : a.n_out + nt * half + (r - half);
    }
    return nt * kTN + r;
  };
  const int64_t e_rows = (int64_t)e * rows_total;
  const char* wexp = reinterpret_cast<const char*>(a.w) + e_rows * G * 16;
  const int bgrp = tid % kSlab;
  uint32_t b_off[kSlab];  // byte offset of this thread's rows at group bgrp
#pragma unroll
  for (int i = 0; i < kSlab; ++i)
    b_off[i] = (uint32_t)global_row(kRowsPerPass * i + tid / kSlab) * (uint32_t)G * 16u +
               (uint32_t)bgrp * 16u;
  // Scales of row tid: kSlab >> gshift bf16 values per slab.
  const char* s_row = reinterpret_cast<const char*>(a.s + (e_rows + global_row(tid)) * gpr);
  static_assert(kSlab == 4, "scale loads below assume 4 groups per slab");

  u32x4_t bs[kSlab];
  u32x2_t ss;
  auto load_slab = [&](int slab) {
    const int sl = min(slab, nslabs - 1);
    const uint32_t step_off = (uint32_t)sl * kSlab * 16u;
#pragma unroll
    for (int i = 0; i < kSlab; ++i)
      bs[i] = *reinterpret_cast<const u32x4_t*>(wexp + (b_off[i] + step_off));
    const char* sp = s_row + ((sl * kSlab) >> gshift) * 2;
    if constexpr (GSHIFT == 0) {
      ss = *reinterpret_cast<const u32x2_t*>(sp);
    } else if constexpr (GSHIFT == 1) {
      ss = u32x2_t{*reinterpret_cast<const uint32_t*>(sp), 0u};
    } else {
      ss = u32x2_t{(uint32_t)*reinterpret_cast<const uint16_t*>(sp), 0u};
    }
  };
  auto store_slab = [&]() {
#pragma unroll
    for (int i = 0; i < kSlab; ++i) {
      unsigned char* d = Bp + (kRowsPerPass * i + tid / kSlab) * kBpitch + bgrp * 16;
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
  const int mcount = (count + 31) >> 5;  // active 32-token blocks (workgroup-uniform)

  struct AStage {
    u32x4_t v[NA];
  };
  // Octet i of a thread holds row (tid + 256 i) / 4: only the octets of the
  // MC active token blocks (rows < 32 MC) are loaded and parked; rows of
  // inactive blocks are never read by the MFMAs.
  auto load_a = [&](AStage& st, int step, auto mc_c) {
    constexpr int NAE = (decltype(mc_c)::value * 32 * 4 + 255) / 256;
    const int k = min(step, G - 1);
#pragma unroll
    for (int i = 0; i < NAE; ++i) st.v[i] = a_src[i][k * 4];
  };
  auto store_a = [&](const AStage& st, unsigned char* Ab, auto mc_c) {
    constexpr int NAE = (decltype(mc_c)::value * 32 * 4 + 255) / 256;
#pragma unroll
    for (int i = 0; i < NAE; ++i) *reinterpret_cast<u32x4_t*>(Ab + a_lds[i]) = st.v[i];
  };
  // Packed words and scale of group g for this lane's two weight rows.
  struct BRaw {
    u32x2_t w[2];
    float s[2];
  };
  auto read_b = [&](BRaw& r, int g) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      r.w[n] = *reinterpret_cast<const u32x2_t*>(Bp + nrow[n] * kBpitch + g * 16 + q * 8);
      r.s[n] = Sc[nrow[n] * kSpitch + g];
    }
  };
  auto dequant_b = [&](const BRaw& r, bf16x8_t (&bfr)[2][2]) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const float b = -8.0f * r.s[n];
      bfr[n][0] = dequant_word(r.w[n][0], r.s[n], b);
      bfr[n][1] = dequant_word(r.w[n][1], r.s[n], b);
    }
  };

  // The main loop for MC active token blocks.  Step s runs its MFMAs with
  // the B fragments dequantized during step s-1 and, interleaved with them,
  // dequantizes step s+1's fragments: the matrix core and the vector ALU work
  // side by side inside one wave.  One barrier per step (the double-buffered
  // activation tile), one more where a new weight slab is parked.
  auto run = [&](auto mc_c) {
    constexpr int MC = decltype(mc_c)::value;
    f32x16_t acc[MC][2];
#pragma unroll
    for (int m = 0; m < MC; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.0f;

    // Prologue: slab 0 and A(0) in LDS, A(1), A(2) and slab 1 in flight.
    // Its loads stay in program order (scheduling barriers), the order the
    // loop issues them in: the wait counts at the loop head merge the first
    // entry with the back edge, and a reordered prologue would leave the
    // loop waiting for every load in flight once per slab.
    AStage st[2];
    load_slab(0);
    __builtin_amdgcn_sched_barrier(0);
    load_a(st[0], 0, mc_c);
    __builtin_amdgcn_sched_barrier(0);
    load_a(st[1], 1, mc_c);
    __builtin_amdgcn_sched_barrier(0);
    store_slab();
    store_a(st[0], A0, mc_c);
    __builtin_amdgcn_sched_barrier(0);
    load_a(st[0], 2, mc_c);
    __builtin_amdgcn_sched_barrier(0);
    load_slab(1);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    bf16x8_t bcur[2][2], bnext[2][2];
    {
      BRaw r0;
      read_b(r0, 0);
      dequant_b(r0, bcur);
    }

    for (int slab = 0; slab < nslabs; ++slab) {
#pragma unroll
      for (int g = 0; g < kSlab; ++g) {
        const int step = slab * kSlab + g;
        unsigned char* const Acur = A0 + (g & 1) * kAbytes;
        unsigned char* const Anext = A0 + ((g + 1) & 1) * kAbytes;
        // A(step+1) into the other buffer (read last in step-1, which every
        // wave has finished), then refill its registers with A(step+3).
        store_a(st[(g + 1) & 1], Anext, mc_c);
        load_a(st[(g + 1) & 1], step + 3, mc_c);
        if (g == kSlab - 1) {
          // Every wave read this slab's last group in step-1: park the next.
          // Unconditional, also after the last slab (a clamped reload whose
          // data is never used): every path to the loop head then carries
          // the same loads, so the waits there stay exact.
          store_slab();
          __syncthreads();
          load_slab(slab + 2);
        }
        // Next step's weight fragments.  Unconditional so that one basic
        // block holds the reads, the MFMAs and the dequantization (after the
        // last step this reads a stale but valid group and is never used).
        BRaw rn;
        read_b(rn, (g + 1) & (kSlab - 1));
#pragma unroll
        for (int m = 0; m < MC; ++m) {
#pragma unroll
          for (int sub = 0; sub < 2; ++sub) {
            const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(
                Acur + (m * 32 + j) * kApitch + (2 * q + sub) * 16);
#pragma unroll
            for (int n = 0; n < 2; ++n)
              acc[m][n] =
                  __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bcur[n][sub], acc[m][n], 0, 0, 0);
          }
        }
        dequant_b(rn, bnext);
        // Interleave: the activation and weight reads first, then each MFMA
        // followed by a share of the dequantization.
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * MC + 4, 0);
#pragma unroll
        for (int i = 0; i < 4 * MC; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 96 / (4 * MC), 0);
        }
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
          for (int h = 0; h < 2; ++h) bcur[n][h] = bnext[n][h];
        __syncthreads();
      }
    }

    // Epilogue.  Accumulator register r of a 32x32 block holds row
    // 8*(r/4) + 4*(lane/32) + r%4 and column lane%32.
#pragma unroll
    for (int m = 0; m < MC; ++m) {
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
          const int col = nt * kTN + 64 * wid + j;
          if (a.partial_bf16) {
            uint16_t* out = static_cast<uint16_t*>(a.out) + (int64_t)f * a.n_out;
            out[col] = (uint16_t)f32_to_bf16(acc[m][0][r] * wt);
            out[col + 32] = (uint16_t)f32_to_bf16(acc[m][1][r] * wt);
          } else {
            float* out = static_cast<float*>(a.out) + (int64_t)f * a.n_out;
            out[col] = acc[m][0][r] * wt;
            out[col + 32] = acc[m][1][r] * wt;
          }
        }
      }
    }
  };

  static_assert(TMB == 4 || TMB == 8, "token tile of 4 or 8 blocks");
  switch (mcount) {
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 2>{}); break;
    case 3: run(std::integral_constant<int, 3>{}); break;
    case 4: run(std::integral_constant<int, 4>{}); break;
    default:
      if constexpr (TMB == 8) {
        switch (mcount) {
          case 5: run(std::integral_constant<int, (TMB == 8 ? 5 : 1)>{}); break;
          case 6: run(std::integral_constant<int, (TMB == 8 ? 6 : 1)>{}); break;
          case 7: run(std::integral_constant<int, (TMB == 8 ? 7 : 1)>{}); break;
          default: run(std::integral_constant<int, (TMB == 8 ? 8 : 1)>{}); break;
        }
      }
      break;
  }
}

template <int MODE, int TMB>
hipError_t launch_mfma_m(const MfmaLaunch& a, hipStream_t stream) {
  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  const int64_t grid = (int64_t)a.max_tiles * (rows_total / kTN);
  if (grid <= 0) return hipSuccess;
  const dim3 g((unsigned)grid), b(256);
  constexpr int lds = lds_bytes<TMB>();
  switch (a.group) {
    case 32: hipLaunchKernelGGL((mfma_kernel<MODE, 0, TMB>), g, b, lds, stream, a); break;
    case 64: hipLaunchKernelGGL((mfma_kernel<MODE, 1, TMB>), g, b, lds, stream, a); break;
    case 128: hipLaunchKernelGGL((mfma_kernel<MODE, 2, TMB>), g, b, lds, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_mfma_t(const MfmaLaunch& a, hipStream_t stream) {
  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  if (rows_total % kTN != 0 || a.kdim % (32 * kSlab) != 0) return hipErrorInvalidValue;
  switch (a.tile_m) {
    case kMfmaTileM: return launch_mfma_m<MODE, kMfmaTileM / 32>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_w13_mfma(const MfmaLaunch& a, hipStream_t stream) {
  return launch_mfma_t<0>(a, stream);
}

hipError_t launch_w2_mfma(const MfmaLaunch& a, hipStream_t stream) {
  return launch_mfma_t<1>(a, stream);
}

}  // namespace w4a16
