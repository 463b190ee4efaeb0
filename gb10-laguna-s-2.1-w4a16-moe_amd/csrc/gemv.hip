// Bandwidth-bound grouped dequant-GEMV kernels for few tokens per expert.
//
// Reference kernels: _w4a16_moe_w1_fused_kernel (kernels/w4a16_moe.py:374-499)
// and _w4a16_moe_w2_kernel (:502-634), which dequantize 64x64 tiles of a
// repacked layout and feed tl.dot.  This file reads the unchanged
// pack-quantized rows instead (one row = one output channel, K contiguous).
//
// Work item = one workgroup of WAVES waves: one 16-slot expert block x
// WAVES slabs of output rows, one slab per wave.  The block's activation rows
// are staged into LDS once by the whole workgroup and shared by its waves.
// Lane layout: 8 lanes per weight row, each lane owns whole 32-element groups
// (one 16-byte dwordx4 = 4 packed words = 32 int4 codes), so the 8 lanes of a
// row read one contiguous 128-byte line per step and the 8 row groups of a
// wave read 8 lines.  Each lane walks groups gi = 8*it + (lane % 8).

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
// computed once when the row is staged; the dot2 chain of a group starts from
// -C, so it ends at P - C.  The scale is applied once per group:
// y += s * (P - C).  Products of bf16 activations with small integers are
// exact in fp32, so the only rounding is fp32 accumulation.
//
// The mask and the magic constant arrive as kernel arguments and the magic is
// copied to a vector register once: as opaque registers (one scalar, one
// vector) they let the compiler fuse each pair into one v_and_or_b32 -- with
// immediate constants it emits a separate AND and OR.
// Weight and scale addresses are 32-bit offsets from per-expert bases held in
// scalar registers.
#include <type_traits>

#include "common.hpp"

namespace w4a16 {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// LDS index of activation octet u (8 bf16 values) in a staged row: one pad
// octet after every 32-element group spreads the 8 lanes of a row over
// distinct banks.  A staged row of G groups is followed by one zero group
// (with C = 0): steps past the row end read it and add exactly nothing.
__device__ __forceinline__ int lds_octet(int u) { return u + (u >> 2); }

__host__ __device__ __forceinline__ int staged_row_octets(int kdim) {
  return 5 * ((kdim >> 5) + 1);
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
// pair order word_dot expects, plus the per-group offset correction C.  NT
// threads take part, thread `tid` (NT a multiple of 64, tid in [0, NT)).
template <int NT>
__device__ __forceinline__ void stage_row(const uint16_t* __restrict__ src, int kdim,
                                          u32x4_t* xp, float* xc, int tid) {
  const int n_oct = kdim >> 3;
  const u32x4_t* s4 = reinterpret_cast<const u32x4_t*>(src);
  // octets n_oct .. n_oct+3 form the zero group
  for (int u0 = 0; u0 < n_oct + 4; u0 += NT) {
    const int u = u0 + tid;
    u32x4_t d = {0u, 0u, 0u, 0u};
    if (u < n_oct) d = s4[u];
    const float x0 = bf16_to_f32(d[0] & 0xFFFFu), x1 = bf16_to_f32(d[0] >> 16);
    const float x2 = bf16_to_f32(d[1] & 0xFFFFu), x3 = bf16_to_f32(d[1] >> 16);
    const float x4 = bf16_to_f32(d[2] & 0xFFFFu), x5 = bf16_to_f32(d[2] >> 16);
    const float x6 = bf16_to_f32(d[3] & 0xFFFFu), x7 = bf16_to_f32(d[3] >> 16);
    float c = -136.0f * (((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7)));
    u32x4_t p;
    p[0] = (d[0] & 0xFFFFu) | (d[2] << 16);      // (x0, x4)
    p[1] = (d[0] >> 16) | (d[2] & 0xFFFF0000u);  // (x1, x5)
    p[2] = (d[1] & 0xFFFFu) | (d[3] << 16);      // (x2, x6)
    p[3] = (d[1] >> 16) | (d[3] & 0xFFFF0000u);  // (x3, x7)
    if (u < n_oct + 4) xp[lds_octet(u)] = p;
    c = quad_sum(c);  // the 4 octets of a group sit in one lane quad
    if (u < n_oct + 4 && (tid & 3) == 0) xc[u >> 2] = c;  // -C
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

#ifndef GEMV_MIN_WAVES
#define GEMV_MIN_WAVES 1
#endif

// Sum over aligned groups of LPR lanes; every lane of the group gets it.
template <int LPR>
__device__ __forceinline__ float lane_group_sum(float v) {
  v = oct_sum(v);
  if constexpr (LPR >= 16) v += dpp_f32<0x140>(v);  // row_mirror: the other 8
  if constexpr (LPR >= 32) v += __shfl_xor(v, 16, 64);
  return v;
}

// Self-routing handles at most this many (token, slot) pairs: four per lane.
constexpr int kRouteMaxTok = 256;

// Position of the k-th set bit of m (k < popcount(m)): binary search on the
// popcount of the lower half.
__device__ __forceinline__ int nth_set_bit(uint64_t m, int k) {
  int pos = 0;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    const uint64_t low = m & ((1ull << s) - 1ull);
    const int c = __popcll(low);
    const bool up = k >= c;
    k -= up ? c : 0;
    m = up ? (m >> s) : low;
    pos += up ? s : 0;
  }
  return pos;
}

// Self-routing in registers, by every wave on its own (no LDS, no barrier).
// Work item `item` is flat slot `item`; it carries work only when that slot
// is the first (lowest flat index) routed to its expert, and then covers all
// of the expert's pairs in ascending flat index -- the order
// moe_align_block_size gives them (kernels/w4a16_moe.py:243-278).  Lane l
// gets in fl[j] the flat index of the expert's pair of rank l + 64 j (n_tok
// past the last).  e_out = -1 when the item has no work; dropped = pairs with
// ids outside [0, E).  Requires 1 <= n_tok <= kRouteMaxTok.
// NQ: ids per lane actually read (1 when n_tok <= 64, else 4); the lanes'
// further ids count as absent.
template <int NQ>
__device__ __forceinline__ void route_wave(const GemvLaunch& a, int item, int& e_out,
                                           int& t_out, int (&fl)[4], int& dropped) {
  const int lane = __lane_id();
  const int n_tok = a.n_tok, E = a.num_experts;
  constexpr int kNone = -2147483647 - 1;
  int id[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {  // clamped loads, all in flight together
    const int f = lane + 64 * q;
    int v = kNone;
    if (q < NQ) v = a.ids[min(f, n_tok - 1)];
    id[q] = f < n_tok ? v : kNone;
  }
  int drop = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    drop += __popcll(ballot(id[q] != kNone && (id[q] < 0 || id[q] >= E)));
  dropped = drop;
#pragma unroll
  for (int j = 0; j < 4; ++j) fl[j] = n_tok;
  e_out = -1;
  t_out = 0;
  const int e = __builtin_amdgcn_readfirstlane(a.ids[item]);
  if (e < 0 || e >= E) return;
  bool earlier = false;
#pragma unroll
  for (int q = 0; q < 4; ++q) earlier |= (lane + 64 * q < item) && id[q] == e;
  if (ballot(earlier) != 0) return;  // an earlier slot's item owns this expert
  uint64_t m[4];
  int c[4];
  int T = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    m[q] = ballot(id[q] == e);
    c[q] = __popcll(m[q]);
    T += c[q];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j * 64 >= T) break;  // uniform
    const int R = lane + 64 * j;
    int p = 0, q_sel = 0, p_sel = 0;
    uint64_t m_sel = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (R >= p && R < p + c[q]) {
        q_sel = q;
        p_sel = p;
        m_sel = m[q];
      }
      p += c[q];
    }
    if (R < T) fl[j] = 64 * q_sel + nth_set_bit(m_sel, R - p_sel);
  }
  e_out = e;
  t_out = T;
}

// MODE 0: w13 rows (gate n, up N+n), epilogue SiLU(gate)*up -> bf16 inter.
// MODE 1: w2 rows, epilogue * topk weight -> partial (bf16, or fp32 at M <= 4).
// RPL:   output rows per lane (w13: gate+up pairs, so 2*RPL weight rows).
// PF:    weight loads kept in flight, in group steps.
// TC:    activation rows staged per pass.
// WAVES: waves per workgroup (row slabs sharing one staged block).
// NIT:   group steps per row (ceil(kdim / 256)) when fixed at compile time,
//        0 for any other length.
// ROUTE: the workgroup routes itself from topk_ids (no align kernel); work
//        item i is the i-th expert with routed pairs, all of its pairs.
template <int MODE, int RPL, int PF, int TC, int WAVES, int NIT, bool ROUTE, int UPW, int LPR>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(GEMV_MIN_WAVES)))
void gemv_kernel(const GemvLaunch a) {
  static_assert(UPW == 1 || (NIT > 0 && NIT % PF == 0), "units per workgroup need unrolled steps");
  static_assert(LPR == 8 || LPR == 16 || LPR == 32, "lanes per row");
  constexpr int NR = MODE == 0 ? 2 * RPL : RPL;  // weight rows per lane
  constexpr int NT = 64 * WAVES;
  constexpr int RG = 64 / LPR;                   // row groups per wave
  extern __shared__ u32x4_t lds[];

  const int rows_per_wave = RG * RPL;
  const int chunks = a.n_out / rows_per_wave;           // row chunks (one wave each)
  const int slabs = (chunks + WAVES - 1) / WAVES;       // slabs of WAVES chunks
  const int groups = (slabs + UPW - 1) / UPW;           // workgroups per item
  const int item = blockIdx.x / groups;
  const int slab0 = (blockIdx.x - item * groups) * UPW; // first of UPW slabs (units)
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Unit u covers chunk (slab0 + u) * WAVES + wid; chunks past the end are
  // re-read from the last chunk and not stored.
  auto unit_chunk = [&](int u, bool& valid) {
    const int c = (slab0 + u) * WAVES + wid;
    valid = c < chunks;  // wave-uniform
    return valid ? c : chunks - 1;
  };
  bool has_rows;
  const int chunk = unit_chunk(0, has_rows);
  const int tid = threadIdx.x;
  const int lane = __lane_id();

  // LDS: staged activation rows | their -C values
  const int G0 = a.kdim >> 5;
  const int row_oct = staged_row_octets(a.kdim);
  const int xc_pitch = G0 + 1;
  u32x4_t* xp = lds;
  float* xc = reinterpret_cast<float*>(lds + TC * row_oct);

  int e, T, f_lane = 0;
  int fl[4];
  if constexpr (ROUTE) {
    int dropped;
    if (a.n_tok <= 64)
      route_wave<1>(a, item, e, T, fl, dropped);
    else
      route_wave<4>(a, item, e, T, fl, dropped);
    if (MODE == 0 && blockIdx.x == 0 && tid == 0) a.dropped_out[0] = dropped;
    if (e < 0) return;  // workgroup-uniform: every wave routes the same item
  } else {
    int blk = item;
    if (a.block_list) {
      if (item >= a.header[3]) return;
      blk = a.block_list[item];
    }
    if (blk * a.block >= a.header[0]) return;
    e = a.expert_ids[blk];
    if (e < 0) return;
    f_lane = lane < a.block ? a.sorted[blk * a.block + lane] : a.n_tok;
    T = __popcll(ballot(f_lane < a.n_tok));  // valid slots are a prefix
  }
  // Flat index of the item's t-th pair (t < T).
  auto slot_of = [&](int t) -> int {
    if constexpr (ROUTE) {
      const int src = t & 63;
      int v = __shfl(fl[0], src, 64);
      if (T > 64) {  // uniform; ranks past 63 sit in fl[1..3]
        const int q = t >> 6;
        const int v1 = __shfl(fl[1], src, 64), v2 = __shfl(fl[2], src, 64);
        const int v3 = __shfl(fl[3], src, 64);
        v = q == 0 ? v : (q == 1 ? v1 : (q == 2 ? v2 : v3));
      }
      return v;
    } else {
      (void)fl;
      return __shfl(f_lane, t, 64);
    }
  };

  const int r = lane / LPR;
  const int sl = lane % LPR;

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
      row = (j < RPL) ? n_base + RG * j : a.n_out + n_base + RG * (j - RPL);
    else
      row = n_base + RG * j;
    woff[j] = (uint32_t)row * (uint32_t)G * 16u;
    soff[j] = (uint32_t)row * (uint32_t)gpr * 2u;
  }

  const int n_it = (G + LPR - 1) / LPR;

  // The whole item for NTOK (compile-time) tokens per pass.  Every variant
  // owns its prefetch ring: sharing one ring between variants lets the
  // register allocator reuse a ring register for activations, after which
  // each step waits for every load in flight.  With NIT > 0 (the step count
  // known at compile time) the step loop is fully unrolled and nothing is in
  // flight across a loop edge, so every wait the compiler places is exact.
  auto body = [&](auto ntok_c) {
    constexpr int NTOK = decltype(ntok_c)::value;
    // Weight and raw bf16 scale registers of PF steps in flight.  Scales
    // stay as raw bits until use: converting right after the load would make
    // the compiler wait for it there and serialise the prefetch ring.
    u32x4_t wb[PF][NR];
    uint32_t sb[PF][NR];
    // Step `it` of unit `u` (unit 0 = this wave's first chunk).
    auto load_step = [&](u32x4_t (&wq)[NR], uint32_t (&sq)[NR], int u, int it) {
      // An opaque step index keeps the address math at this point: with a
      // constant index the compiler computes every step's addresses up front
      // and holds them in registers.
      asm volatile("" : "+s"(it));
      const uint32_t gi = (uint32_t)min(it * LPR + sl, G - 1);
      uint32_t dw = 0, ds = 0;  // unit offsets from unit 0 (wave-uniform)
      if (UPW > 1 && u > 0) {
        bool v;
        const uint32_t drow = (uint32_t)((unit_chunk(u, v) - chunk) * rows_per_wave);
        dw = drow * (uint32_t)G * 16u;
        ds = drow * (uint32_t)gpr * 2u;
      }
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        wq[j] = *reinterpret_cast<const u32x4_t*>(wexp + (woff[j] + dw + gi * 16u));
        sq[j] = *reinterpret_cast<const uint16_t*>(sexp + (soff[j] + ds + (gi >> gshift) * 2u));
      }
    };
    // One group step: 8 lanes per row, lane sl on group 8*it + sl; steps past
    // the row end meet the zero activation group and add nothing.
    auto compute_step = [&](const u32x4_t (&wq)[NR], const uint32_t (&sq)[NR], int it,
                            float (&acc)[NR][NTOK]) {
      const int gi = it * LPR + sl;
      const int gl = gi < G ? gi : G;
      float pj[NR][NTOK];
#pragma unroll
      for (int t = 0; t < NTOK; ++t) {
        const float c = xc[t * xc_pitch + gl];  // -C
#pragma unroll
        for (int j = 0; j < NR; ++j) pj[j][t] = c;
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        u32x4_t x[NTOK];
#pragma unroll
        for (int t = 0; t < NTOK; ++t) x[t] = xp[t * row_oct + lds_octet(gl * 4 + w)];
#pragma unroll
        for (int j = 0; j < NR; ++j) {
          const uint32_t wv = wq[j][w];
          const uint32_t d0 = (wv & mask) | magic;
          const uint32_t d1 = ((wv >> 4) & mask) | magic;
          const uint32_t d2 = ((wv >> 8) & mask) | magic;
          const uint32_t d3 = ((wv >> 12) & mask) | magic;
#pragma unroll
          for (int t = 0; t < NTOK; ++t) {
            float q = dot2(d0, x[t][0], pj[j][t]);
            q = dot2(d1, x[t][1], q);
            q = dot2(d2, x[t][2], q);
            pj[j][t] = dot2(d3, x[t][3], q);
          }
        }
        // One word's activation reads at a time (NTOK * 4 registers); the
        // other waves of the SIMD cover the LDS latency.
        if (NTOK > 1) __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const float sc = bf16_to_f32(sq[j]);
#pragma unroll
        for (int t = 0; t < NTOK; ++t) {
          acc[j][t] = fmaf(sc, pj[j][t], acc[j][t]);
          // Pin the step's math here: left alone, the compiler sinks it
          // towards the final reduction and keeps every loaded step alive.
          asm volatile("" : "+v"(acc[j][t]));
        }
      }
    };

    for (int t0 = 0; t0 < T; t0 += NTOK) {
      const int tc = min(NTOK, T - t0);  // tokens past tc compute unused values
      // w2: the pair this lane stores and its routing weight, loaded here so
      // that the load overlaps the weight stream instead of ending it.  (w13
      // finds its pair only at the end: one more live register there would
      // cost its 4-token variant a wave per SIMD.)
      const int f_pre = MODE == 1 ? slot_of(min(t0 + sl, T - 1)) : 0;
      const float wt_mine = MODE == 1 ? a.topk_w[f_pre] : 0.0f;
      // Opaque row offsets per pass: otherwise every load address of the pass
      // is loop-invariant, gets hoisted out of the pass loop and stays live
      // in registers for the whole kernel.
#pragma unroll
      for (int j = 0; j < NR; ++j) asm volatile("" : "+v"(woff[j]), "+v"(soff[j]));

#pragma unroll
      for (int p = 0; p < PF; ++p)
        if (NIT == 0 || p < UPW * NIT) {
          constexpr int kN = NIT > 0 ? NIT : 1;
          load_step(wb[p], sb[p], NIT ? p / kN : 0, NIT ? p % kN : min(p, n_it - 1));
        }

      // Stage this pass's activation rows (the whole workgroup).
      __syncthreads();
      for (int t = 0; t < tc; ++t) {
        const int f = slot_of(t0 + t);
        const int64_t arow = MODE == 0 ? f / a.topk : f;
        stage_row<NT>(a.act + arow * a.ld_act, kdim, xp + t * row_oct, xc + t * xc_pitch,
                      tid);
      }
      __syncthreads();

      float acc[NR][NTOK];
      auto clear = [&]() {
#pragma unroll
        for (int j = 0; j < NR; ++j)
#pragma unroll
          for (int t = 0; t < NTOK; ++t) acc[j][t] = 0.0f;
      };
      // Reduce each row over its 8 lanes; lane sl then owns token t0+sl.
      auto finish = [&](int u) {
#pragma unroll
        for (int j = 0; j < NR; ++j)
#pragma unroll
          for (int t = 0; t < NTOK; ++t) acc[j][t] = lane_group_sum<LPR>(acc[j][t]);
        bool valid;
        const int cu = unit_chunk(u, valid);
        const int nb = cu * rows_per_wave + r;
        const int f_mine = MODE == 1 ? f_pre : slot_of(min(t0 + sl, T - 1));
        if (valid && sl < tc) {
          float v[NR];
#pragma unroll
          for (int j = 0; j < NR; ++j) {
            v[j] = acc[j][0];
#pragma unroll
            for (int t = 1; t < NTOK; ++t)
              if (sl == t) v[j] = acc[j][t];
          }
          if (MODE == 0) {
            uint16_t* out = static_cast<uint16_t*>(a.out) + (int64_t)f_mine * a.n_out;
#pragma unroll
            for (int q = 0; q < RPL; ++q)
              out[nb + RG * q] = (uint16_t)f32_to_bf16(silu(v[q]) * v[RPL + q]);
          } else {
            const float wt = wt_mine;
            if (a.partial_bf16) {
              uint16_t* out = static_cast<uint16_t*>(a.out) + (int64_t)f_mine * a.n_out;
#pragma unroll
              for (int q = 0; q < RPL; ++q) out[nb + RG * q] = (uint16_t)f32_to_bf16(v[q] * wt);
            } else {
              float* out = static_cast<float*>(a.out) + (int64_t)f_mine * a.n_out;
#pragma unroll
              for (int q = 0; q < RPL; ++q) out[nb + RG * q] = v[q] * wt;
            }
          }
        }
      };

      if constexpr (NIT > 0) {
        // UPW units back to back: the prefetch ring runs on across unit
        // boundaries, so a unit's first steps are in flight while the
        // previous unit finishes.
#pragma unroll
        for (int s = 0; s < UPW * NIT; ++s) {
          const int u = s / NIT, it = s % NIT;
          if (it == 0) clear();
          compute_step(wb[s % PF], sb[s % PF], it, acc);
          if (s + PF < UPW * NIT) load_step(wb[s % PF], sb[s % PF], (s + PF) / NIT, (s + PF) % NIT);
          // Straight-line code: keep each step's loads behind the earlier
          // steps' math, or the scheduler hoists them all and the registers
          // they hold cost occupancy.
          __builtin_amdgcn_sched_barrier(0);
          if (it == NIT - 1) finish(u);
        }
      } else {
        // Step count known only at run time: loads stay unconditional (steps
        // past the row end re-read the last group's line, a cache hit) so
        // the same number of loads is in flight on every path.
        clear();
        for (int it0 = 0; it0 < n_it; it0 += PF) {
#pragma unroll
          for (int p = 0; p < PF; ++p) {
            const int it = it0 + p;
            if (it < n_it) compute_step(wb[p], sb[p], it, acc);  // wave-uniform
            load_step(wb[p], sb[p], 0, min(it + PF, n_it - 1));
          }
        }
        finish(0);
      }
    }
  };

  // One variant per block: T >= TC runs passes of TC tokens.
  const int tcap = min(T, TC);
  if (TC >= 4 && tcap >= 4) body(std::integral_constant<int, (TC >= 4 ? 4 : 1)>{});
  else if (TC >= 3 && tcap == 3) body(std::integral_constant<int, (TC >= 3 ? 3 : 1)>{});
  else if (TC >= 2 && tcap == 2) body(std::integral_constant<int, (TC >= 2 ? 2 : 1)>{});
  else body(std::integral_constant<int, 1>{});
}

// The w2 GEMV and the top-k combine of a few-token call in one launch.
//
// A workgroup has one wave per slot (topk <= 16) and owns 8 output rows of
// one token (blockIdx.y); an expert routed from several tokens is read once
// per token.
// Wave t computes slot t's 8 rows exactly as gemv_kernel<1, ...> does (8
// lanes per row on groups 8*it + lane%8, the same dot2 chain per word and
// fma per group, the same 8-lane sum), multiplies by the routing weight and
// parks the value in LDS.  The workgroup then adds the slots in order from
// 0.0, skipping ids outside [0, E), as combine_kernel does.  The result is
// therefore bit-identical to gemv_kernel + combine_kernel (with the same
// bf16 rounding of each weighted slot value when the call keeps bf16 partial
// rows), with one launch, no partial rows in memory, and every wave's weight
// loads in flight at once.
template <int NIT>
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
  float* red = reinterpret_cast<float*>(lds + topk * row_oct) + topk * (G + 1);  // [topk][8]

  const int E = a.num_experts;
  const int e_raw = a.ids[f];
  const float wt = a.topk_w[f];  // loaded with the id, used at the end
  const bool valid = e_raw >= 0 && e_raw < E;  // wave-uniform
  const int e = valid ? e_raw : 0;
  stage_row<64>(a.act + (int64_t)f * a.ld_act, kdim, xp, xc, lane);

  const int r = lane >> 3, sl = lane & 7;
  const int row = blockIdx.x * 8 + r;
  const char* wrow = reinterpret_cast<const char*>(a.w) + ((int64_t)e * a.n_out + row) * G * 16;
  const char* srow = reinterpret_cast<const char*>(a.s) + ((int64_t)e * a.n_out + row) * gpr * 2;
  const uint32_t mask = a.nib_mask;
  uint32_t magic;
  asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "s"(a.nib_magic));
  const int n_it = NIT > 0 ? NIT : (G + 7) >> 3;
  constexpr int kMaxIt = NIT > 0 ? NIT : 1;

  // All loads first (NIT of them), then the staged row is ready.
  u32x4_t wq[kMaxIt];
  uint32_t sq[kMaxIt];
  if constexpr (NIT > 0) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int gi = min(it * 8 + sl, G - 1);
      wq[it] = *reinterpret_cast<const u32x4_t*>(wrow + gi * 16);
      sq[it] = *reinterpret_cast<const uint16_t*>(srow + (gi >> gshift) * 2);
    }
  }
  __syncthreads();

  float acc = 0.0f;
  auto step = [&](const u32x4_t& w4, uint32_t sbits, int it) {
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
  if constexpr (NIT > 0) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) step(wq[it], sq[it], it);
  } else {
    for (int it = 0; it < n_it; ++it) {
      const int gi = min(it * 8 + sl, G - 1);
      const u32x4_t w4 = *reinterpret_cast<const u32x4_t*>(wrow + gi * 16);
      const uint32_t sb = *reinterpret_cast<const uint16_t*>(srow + (gi >> gshift) * 2);
      step(w4, sb, it);
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
  if (sl == 0) red[t * 8 + r] = valid ? v : 0.0f;
  __syncthreads();
  if (threadIdx.x < 8) {
    float sum = 0.0f;
    for (int s = 0; s < topk; ++s) sum += red[s * 8 + threadIdx.x];
    out[(int64_t)m * ld_out + blockIdx.x * 8 + threadIdx.x] = (uint16_t)f32_to_bf16(sum);
  }
}

size_t w2_token_lds_bytes(int topk, int kdim) {
  return (size_t)topk * (staged_row_octets(kdim) * sizeof(u32x4_t) +
                         (size_t)((kdim >> 5) + 1) * sizeof(float)) +
         (size_t)topk * 8 * sizeof(float);
}

// The staged rows must fit the 64 KB of LDS a workgroup may use.
constexpr size_t kMaxLds = 65536;
#ifndef W4A16_GEMV_WAVES
#define W4A16_GEMV_WAVES 4
#endif
constexpr int kGemvWaves = W4A16_GEMV_WAVES;

size_t gemv_lds_bytes(int tc, int kdim) {
  const size_t row_oct = (size_t)staged_row_octets(kdim);
  return tc * (row_oct * sizeof(u32x4_t) + (size_t)((kdim >> 5) + 1) * sizeof(float));
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
  const size_t lds = gemv_lds_bytes(TC, a.kdim);
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

// M == 1 routes one pair per expert; up to M*topk <= E most touched experts
// get one or two pairs; beyond that stage four rows per pass.
int pick_tc(const GemvLaunch& a, int num_experts) {
  const int M = a.n_tok / a.topk;
  // Measured on MI355X (E=256, top-10): from M = 8 up, four token rows per
  // pass let the experts with 3-4 pairs finish in one pass (M=16: 137 vs
  // 141 us uniform, 105 vs 120 us skewed routing).
  (void)num_experts;
  int tc = 4;
  if (a.tc > 0)
    tc = a.tc;
  else if (M <= 1)
    tc = 1;
  else if (M < 8)
    tc = 2;
  while (tc > 1 && gemv_lds_bytes(tc, a.kdim) > kMaxLds) tc >>= 1;
  return tc;
}

}  // namespace

// Launch shapes: output rows per lane (RPL) and prefetch depth (PF) of the
// two GEMVs, waves per workgroup.  Overridable at build time for tuning sweeps.
#ifndef W4A16_W13_RPL
#define W4A16_W13_RPL 1
#endif
#ifndef W4A16_W13_PF
#define W4A16_W13_PF 4
#endif
#ifndef W4A16_W2_RPL
#define W4A16_W2_RPL 2
#endif
#ifndef W4A16_W2_PF
#define W4A16_W2_PF 2
#endif

// Lanes per weight row: a.lpr, or by default 32 for the w13 launch of
// one-token passes (M = 1), which is short of loads in flight -- 32 lanes per
// row put a whole K = 3072 row's loads in flight at once (M=1: 12.0 -> 11.0
// us) -- and 8 otherwise (whole 128-byte lines per step, the fewest lanes
// per byte; w2's short rows would become many tiny workgroups: 6.8 -> 8.3
// us).  32 exists for passes of 1 or 2 tokens.
int pick_lpr(const GemvLaunch& a, int tc, int mode) {
  if (tc > 2) return 8;
  if (a.lpr > 0) return a.lpr == 32 ? 32 : 8;
  return (mode == 0 && tc == 1) ? 32 : 8;
}

template <int MODE, int R, int P>
hipError_t launch_gemv_tc(const GemvLaunch& a, hipStream_t stream) {
  const int tc = pick_tc(a, a.num_experts);
  const bool wide = pick_lpr(a, tc, MODE) == 32;
  switch (tc) {
    case 1: return wide ? launch_gemv_t<MODE, R, P, 1, 32>(a, stream)
                        : launch_gemv_t<MODE, R, P, 1>(a, stream);
    case 2: return wide ? launch_gemv_t<MODE, R, P, 2, 32>(a, stream)
                        : launch_gemv_t<MODE, R, P, 2>(a, stream);
    default: return launch_gemv_t<MODE, R, P, 4>(a, stream);
  }
}

hipError_t launch_w13_gemv(const GemvLaunch& a_in, hipStream_t stream) {
  GemvLaunch a = a_in;
  a.nib_mask = 0x000F000Fu;
  a.nib_magic = 0x43004300u;  // bf16 (128, 128)
  return launch_gemv_tc<0, W4A16_W13_RPL, W4A16_W13_PF>(a, stream);
}

bool gemv_route_fits(int n_tok, int num_experts, int K, int N) {
  (void)num_experts;
  return n_tok >= 1 && n_tok <= kRouteMaxTok && gemv_lds_bytes(1, K) <= kMaxLds &&
         gemv_lds_bytes(1, N) <= kMaxLds;
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
  const dim3 grid((unsigned)(a.n_out / 8), (unsigned)M), block(64 * a.topk);
  const size_t lds = w2_token_lds_bytes(a.topk, a.kdim);
  const int n_it = ((a.kdim >> 5) + 7) >> 3;
  if (n_it == 4)
    hipLaunchKernelGGL(w2_token_kernel<4>, grid, block, lds, stream, a, out, ld_out);
  else
    hipLaunchKernelGGL(w2_token_kernel<0>, grid, block, lds, stream, a, out, ld_out);
  return hipGetLastError();
}

hipError_t launch_w2_gemv(const GemvLaunch& a_in, hipStream_t stream) {
  GemvLaunch a = a_in;
  a.nib_mask = 0x000F000Fu;
  a.nib_magic = 0x43004300u;
  return launch_gemv_tc<1, W4A16_W2_RPL, W4A16_W2_PF>(a, stream);
}

}  // namespace w4a16
