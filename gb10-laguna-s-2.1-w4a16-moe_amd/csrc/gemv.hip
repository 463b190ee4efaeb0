// Bandwidth-bound grouped dequant-GEMV kernels for few tokens per expert.
//
// Reference kernels: _w4a16_moe_w1_fused_kernel (kernels/w4a16_moe.py:374-499)
// and _w4a16_moe_w2_kernel (:502-634), which dequantize 64x64 tiles of a
// repacked layout and feed tl.dot.  This file reads the unchanged
// pack-quantized rows instead (one row = one output channel, K contiguous).
//
// Work item = one wave: one 16-slot expert block x a slab of output rows.
// Lane layout: 8 lanes per weight row, each lane owns whole 32-element groups
// (one 16-byte dwordx4 = 4 packed words = 32 int4 codes), so the 8 lanes of a
// row read one contiguous 128-byte line per step and the 8 row groups of a
// wave read 8 lines.  Each lane walks groups gi = 8*it + (lane % 8).
//
// Dequantisation never forms (code-8)*scale per weight.  A packed word w holds
// codes n0..n7 for k = 8j..8j+7 (nibble i at bits 4i).  One AND-OR per pair
// (after a shift) makes bf16 pairs of value 128 + code:
//   (w       & 0x000F000F) | 0x43004300 -> (128+n0, 128+n4)
//   (w >>  4 & 0x000F000F) | 0x43004300 -> (128+n1, 128+n5)
//   (w >>  8 & 0x000F000F) | 0x43004300 -> (128+n2, 128+n6)
//   (w >> 12 & 0x000F000F) | 0x43004300 -> (128+n3, 128+n7)
// (0x4300 is bf16 128, whose mantissa step is 1.)  v_dot2_f32_bf16 against
// the matching activation pairs (x0,x4) (x1,x5) (x2,x6) (x3,x7) accumulates
//   P = sum_k (code_k + 128) x_k
// and the group's true partial sum is P - C with C = 136 * sum_k x_k, because
// the weight is code - 8.  C depends on the activation row only and is
// computed once when the row is staged.  The scale is applied once per group:
// y += s * (P - C).  Products of bf16 activations with small integers are
// exact in fp32, so the only rounding is fp32 accumulation.
//
// The mask and the magic constant arrive as kernel arguments and the magic is
// copied to a vector register once: as opaque registers (one scalar, one
// vector) they let the compiler fuse each pair into one v_and_or_b32 -- with
// immediate constants it emits a separate AND and OR.
// Weight and scale addresses are 32-bit offsets from per-expert bases held in
// scalar registers.
#include "common.hpp"

namespace w4a16 {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// LDS index of activation octet u (8 bf16 values) in a staged row: one pad
// octet after every 32-element group spreads the 8 lanes of a row over
// distinct banks.
__device__ __forceinline__ int lds_octet(int u) { return u + (u >> 2); }

__device__ __forceinline__ int staged_row_octets(int kdim) {
  return (kdim >> 3) + (kdim >> 5);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

// Sum over one packed word (8 codes) against its permuted activation octet.
__device__ __forceinline__ float word_dot(uint32_t w, const u32x4_t& x, float acc,
                                          uint32_t mask, uint32_t magic) {
  acc = dot2((w & mask) | magic, x[0], acc);
  acc = dot2(((w >> 4) & mask) | magic, x[1], acc);
  acc = dot2(((w >> 8) & mask) | magic, x[2], acc);
  acc = dot2(((w >> 12) & mask) | magic, x[3], acc);
  return acc;
}

// Stage one bf16 activation row of kdim values into LDS, permuted into the
// pair order word_dot expects, plus the per-group offset correction C.
__device__ __forceinline__ void stage_row(const uint16_t* __restrict__ src,
                                          int kdim, u32x4_t* xp, float* xc) {
  const int lane = __lane_id();
  const int n_oct = kdim >> 3;
  const u32x4_t* s4 = reinterpret_cast<const u32x4_t*>(src);
  for (int u0 = 0; u0 < n_oct; u0 += 64) {
    const int u = u0 + lane;
    u32x4_t d = {0u, 0u, 0u, 0u};
    if (u < n_oct) d = s4[u];
    const float x0 = bf16_to_f32(d[0] & 0xFFFFu), x1 = bf16_to_f32(d[0] >> 16);
    const float x2 = bf16_to_f32(d[1] & 0xFFFFu), x3 = bf16_to_f32(d[1] >> 16);
    const float x4 = bf16_to_f32(d[2] & 0xFFFFu), x5 = bf16_to_f32(d[2] >> 16);
    const float x6 = bf16_to_f32(d[3] & 0xFFFFu), x7 = bf16_to_f32(d[3] >> 16);
    float c = 136.0f * (((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7)));
    u32x4_t p;
    p[0] = (d[0] & 0xFFFFu) | (d[2] << 16);      // (x0, x4)
    p[1] = (d[0] >> 16) | (d[2] & 0xFFFF0000u);  // (x1, x5)
    p[2] = (d[1] & 0xFFFFu) | (d[3] << 16);      // (x2, x6)
    p[3] = (d[1] >> 16) | (d[3] & 0xFFFF0000u);  // (x3, x7)
    if (u < n_oct) xp[lds_octet(u)] = p;
    c = quad_sum(c);  // the 4 octets of a group sit in one lane quad
    if (u < n_oct && (lane & 3) == 0) xc[u >> 2] = c;
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// MODE 0: w13 rows (gate n, up N+n), epilogue SiLU(gate)*up -> bf16 inter.
// MODE 1: w2 rows, epilogue * topk weight -> fp32 partial.
// RPL: output rows per lane (w13: gate+up pairs, so 2*RPL weight rows).
// PF:  weight loads kept in flight, in groups-steps.
// TC:  activation rows staged per pass.
template <int MODE, int RPL, int PF, int TC>
__global__ __launch_bounds__(64) void gemv_kernel(const GemvLaunch a) {
  constexpr int NR = MODE == 0 ? 2 * RPL : RPL;  // weight rows per lane
  extern __shared__ u32x4_t lds[];

  const int rows_per_wave = 8 * RPL;
  const int chunks = a.n_out / rows_per_wave;
  const int item = blockIdx.x / chunks;
  const int chunk = blockIdx.x - item * chunks;
  int blk = item;
  if (a.block_list) {
    if (item >= a.header[3]) return;
    blk = a.block_list[item];
  }
  if (blk * a.block >= a.header[0]) return;
  const int e = a.expert_ids[blk];
  if (e < 0) return;

  const int lane = __lane_id();
  const int r = lane >> 3;
  const int sl = lane & 7;

  const int f_lane = lane < a.block ? a.sorted[blk * a.block + lane] : a.n_tok;
  const int T = __popcll(ballot(f_lane < a.n_tok));  // valid slots are a prefix

  const int kdim = a.kdim;
  const int G = kdim >> 5;               // 32-element groups per row
  const int gpr = kdim / a.group;        // scales per row
  const int gshift = a.group == 32 ? 0 : (a.group == 64 ? 1 : 2);
  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  const int n_base = chunk * rows_per_wave + r;
  // The magic constant lives in a VGPR: v_and_or_b32 may read only one scalar
  // operand, so with both constants in SGPRs the compiler would split it.
  const uint32_t mask = a.nib_mask;
  uint32_t magic;
  asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "s"(a.nib_magic));

  // Uniform per-expert bases, per-lane 32-bit row offsets (one expert's rows
  // span well under 4 GB).
  const char* wexp = reinterpret_cast<const char*>(a.w) + (int64_t)e * rows_total * G * 16;
  const char* sexp = reinterpret_cast<const char*>(a.s) + (int64_t)e * rows_total * gpr * 2;
  uint32_t woff[NR], soff[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    int row;
    if (MODE == 0)
      row = (j < RPL) ? n_base + 8 * j : a.n_out + n_base + 8 * (j - RPL);
    else
      row = n_base + 8 * j;
    woff[j] = (uint32_t)row * (uint32_t)G * 16u;
    soff[j] = (uint32_t)row * (uint32_t)gpr * 2u;
  }

  const int row_oct = staged_row_octets(kdim);
  u32x4_t* xp = lds;
  float* xc = reinterpret_cast<float*>(lds + TC * row_oct);
  const int n_it = (G + 7) >> 3;

  for (int t0 = 0; t0 < T; t0 += TC) {
    const int tc = min(TC, T - t0);

    // Weight and raw bf16 scale registers of PF steps in flight.  Scales
    // stay as raw bits until use: converting right after the load would make
    // the compiler wait for it there and serialise the prefetch ring.
    u32x4_t wb[PF][NR];
    uint32_t sb[PF][NR];
    // Loads are unconditional so the waitcnt pass sees the same number of
    // loads in flight on every path: steps past the row end re-read the last
    // step's lines (cache hits) and their results are never used.
    auto load_step = [&](u32x4_t (&wq)[NR], uint32_t (&sq)[NR], int it) {
      const uint32_t gi = (uint32_t)min(min(it, n_it - 1) * 8 + sl, G - 1);
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        wq[j] = *reinterpret_cast<const u32x4_t*>(wexp + (woff[j] + gi * 16u));
        sq[j] = *reinterpret_cast<const uint16_t*>(sexp + (soff[j] + (gi >> gshift) * 2u));
      }
    };
#pragma unroll
    for (int p = 0; p < PF; ++p) load_step(wb[p], sb[p], p);

    // Stage this pass's activation rows.
    __syncthreads();
    for (int t = 0; t < tc; ++t) {
      const int f = __shfl(f_lane, t0 + t, 64);
      const int64_t arow = MODE == 0 ? f / a.topk : f;
      stage_row(a.act + arow * a.ld_act, kdim, xp + t * row_oct, xc + t * G);
    }
    __syncthreads();

    float acc[NR][TC];
#pragma unroll
    for (int j = 0; j < NR; ++j)
#pragma unroll
      for (int t = 0; t < TC; ++t) acc[j][t] = 0.0f;

    for (int it0 = 0; it0 < n_it; it0 += PF) {
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        const int it = it0 + p;
        if (it < n_it) {  // wave-uniform; no loads inside
          const int gi = it * 8 + sl;
          const bool in = gi < G;
          const int gl = in ? gi : G - 1;
#pragma unroll
          for (int t = 0; t < TC; ++t) {
            if (t < tc) {
              const u32x4_t* xg = xp + t * row_oct + lds_octet(gl * 4);
              const u32x4_t x0 = xg[0], x1 = xg[1], x2 = xg[2], x3 = xg[3];
              const float c = xc[t * G + gl];
#pragma unroll
              for (int j = 0; j < NR; ++j) {
                float pj = word_dot(wb[p][j][0], x0, 0.0f, mask, magic);
                pj = word_dot(wb[p][j][1], x1, pj, mask, magic);
                pj = word_dot(wb[p][j][2], x2, pj, mask, magic);
                pj = word_dot(wb[p][j][3], x3, pj, mask, magic);
                const float sc = in ? bf16_to_f32(sb[p][j]) : 0.0f;
                acc[j][t] = fmaf(sc, pj - c, acc[j][t]);
              }
            }
          }
        }
        load_step(wb[p], sb[p], it + PF);
      }
    }

    // Reduce each row over its 8 lanes; lane sl then owns token t0+sl.
#pragma unroll
    for (int j = 0; j < NR; ++j)
#pragma unroll
      for (int t = 0; t < TC; ++t) acc[j][t] = oct_sum(acc[j][t]);

    const int f_mine = __shfl(f_lane, min(t0 + sl, 63), 64);
    if (sl < tc) {
      float v[NR];
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        v[j] = acc[j][0];
#pragma unroll
        for (int t = 1; t < TC; ++t)
          if (sl == t) v[j] = acc[j][t];
      }
      if (MODE == 0) {
        uint16_t* out = static_cast<uint16_t*>(a.out) + (int64_t)f_mine * a.n_out;
#pragma unroll
        for (int q = 0; q < RPL; ++q)
          out[n_base + 8 * q] = (uint16_t)f32_to_bf16(silu(v[q]) * v[RPL + q]);
      } else {
        const float wt = a.topk_w[f_mine];
        float* out = static_cast<float*>(a.out) + (int64_t)f_mine * a.n_out;
#pragma unroll
        for (int q = 0; q < RPL; ++q) out[n_base + 8 * q] = v[q] * wt;
      }
    }
  }
}

// The staged rows must fit the 64 KB of LDS a workgroup may use.
constexpr size_t kMaxLds = 65536;

size_t gemv_lds_bytes(int tc, int kdim) {
  const size_t row_oct = (size_t)(kdim >> 3) + (kdim >> 5);
  return tc * (row_oct * sizeof(u32x4_t) + (size_t)(kdim >> 5) * sizeof(float));
}

template <int MODE, int RPL, int PF, int TC>
hipError_t launch_gemv_t(const GemvLaunch& a, hipStream_t stream) {
  const int rows_per_wave = 8 * RPL;
  if (a.n_out % rows_per_wave != 0) return hipErrorInvalidValue;
  const int chunks = a.n_out / rows_per_wave;
  const size_t lds = gemv_lds_bytes(TC, a.kdim);
  if (lds > kMaxLds) return hipErrorInvalidValue;
  const int64_t grid = (int64_t)a.max_blocks * chunks;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL((gemv_kernel<MODE, RPL, PF, TC>), dim3((unsigned)grid), dim3(64),
                     lds, stream, a);
  return hipGetLastError();
}

// M == 1 routes one pair per expert; up to M*topk <= E most touched experts
// get one or two pairs; beyond that stage four rows per pass.
int pick_tc(const GemvLaunch& a, int num_experts) {
  const int M = a.n_tok / a.topk;
  int tc = 4;
  if (M <= 1)
    tc = 1;
  else if (a.n_tok <= num_experts)
    tc = 2;
  while (tc > 1 && gemv_lds_bytes(tc, a.kdim) > kMaxLds) tc >>= 1;
  return tc;
}

}  // namespace

// Launch shapes: output rows per lane (RPL) and prefetch depth (PF) of the
// two GEMVs.  Overridable at build time for tuning sweeps.
#ifndef W4A16_W13_RPL
#define W4A16_W13_RPL 2
#endif
#ifndef W4A16_W13_PF
#define W4A16_W13_PF 3
#endif
#ifndef W4A16_W2_RPL
#define W4A16_W2_RPL 4
#endif
#ifndef W4A16_W2_PF
#define W4A16_W2_PF 2
#endif

hipError_t launch_w13_gemv(const GemvLaunch& a_in, hipStream_t stream) {
  GemvLaunch a = a_in;
  a.nib_mask = 0x000F000Fu;
  a.nib_magic = 0x43004300u;  // bf16 (128, 128)
  constexpr int R = W4A16_W13_RPL, P = W4A16_W13_PF;
  switch (pick_tc(a, a.num_experts)) {
    case 1: return launch_gemv_t<0, R, P, 1>(a, stream);
    case 2: return launch_gemv_t<0, R, P, 2>(a, stream);
    default: return launch_gemv_t<0, R, P, 4>(a, stream);
  }
}

hipError_t launch_w2_gemv(const GemvLaunch& a_in, hipStream_t stream) {
  GemvLaunch a = a_in;
  a.nib_mask = 0x000F000Fu;
  a.nib_magic = 0x43004300u;
  constexpr int R = W4A16_W2_RPL, P = W4A16_W2_PF;
  switch (pick_tc(a, a.num_experts)) {
    case 1: return launch_gemv_t<1, R, P, 1>(a, stream);
    case 2: return launch_gemv_t<1, R, P, 2>(a, stream);
    default: return launch_gemv_t<1, R, P, 4>(a, stream);
  }
}

}  // namespace w4a16
