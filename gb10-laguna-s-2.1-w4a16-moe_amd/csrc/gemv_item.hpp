// Bandwidth-bound grouped dequant-GEMV work items for few tokens per expert
// (device code shared by the GEMV-only launches and the mixed GEMV + MFMA
// launches).
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
#pragma once

#include <type_traits>

#include "common.hpp"

namespace w4a16 {
namespace {
namespace gemv_dev {

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

// Octet u of a staged row (below) from its loaded bits d, zero past the
// row: every lane of the wave calls it (the -C sum crosses a lane quad).
__device__ __forceinline__ void stage_octet(u32x4_t d, int u, int n_oct, u32x4_t* xp, float* xc,
                                            int tid) {
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
    stage_octet(d, u, n_oct, xp, xc, tid);
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }


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

// Self-routing, by every wave on its own (no barrier).  A work item covers
// all of one expert's pairs in ascending flat index -- the order
// moe_align_block_size gives them (kernels/w4a16_moe.py:243-278).  Lane l
// gets in fl[j] the flat index of the expert's pair of rank l + 64 j (n_tok
// past the last).  e_out = -1 when the item has no work; dropped = pairs
// with ids outside [0, E).  Requires 1 <= n_tok <= kRouteMaxTok.
// By default work item `item` is flat slot `item`, with work when that slot
// is the first routed to its expert (one ballot).  COMPACT (the w13 launch)
// from 65 pairs, where many slots repeat an earlier slot's expert: work item
// `item` is the item-th first slot in flat order, so the items with work fill
// the start of the grid and the empty ones (past the number of routed
// experts) its end, where they hold a slot in the launch's tail rather than
// among the streaming workgroups: M=16 123.0 -> 121.8 us per call, M=12
// 102.8 -> 102.2, skewed M=8, 12, 16 57.2 -> 56.1, 72.4 -> 70.8, 93.2 ->
// 91.8.  Below 65 pairs the search cost more than the few empty items
// (M=2 25.9 -> 26.6).  tab: this wave's E ints of LDS, where the first slot
// of every expert is a minimum over the slots (a wave's LDS instructions run
// in order, so no wait separates the steps).
// FROM_ITEMS (the w2 launch, after a w13 launch that wrote a.route_items):
// item `item` is w13's item `item`, whose expert (-1: no work) the w13
// launch left in a.route_items; the same search on w2's shorter workgroups
// cost more than it saved (uniform M=8, 12, 16: +1.0, +1.5, +0.2 us).
// NQ: ids per lane actually read (1 when n_tok <= 64, else 4); the lanes'
// further ids count as absent.
template <int NQ, bool COMPACT, bool FROM_ITEMS>
__device__ __forceinline__ void route_wave(const GemvLaunch& a, int item, int& e_out,
                                           int& t_out, int (&fl)[4], int& dropped, int* tab) {
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
  int e;
  if (FROM_ITEMS) {
    e = __builtin_amdgcn_readfirstlane(a.route_items[item]);
    if (e < 0 || e >= E) return;
  } else if (!COMPACT || NQ == 1 || n_tok <= a.topk) {
    e = __builtin_amdgcn_readfirstlane(a.ids[item]);
    if (e < 0 || e >= E) return;
    bool earlier = false;
#pragma unroll
    for (int q = 0; q < NQ; ++q) earlier |= (lane + 64 * q < item) && id[q] == e;
    if (ballot(earlier) != 0) return;  // an earlier slot's item owns this expert
  } else {
    auto valid = [&](int v) { return v >= 0 && v < E; };
    for (int x = lane; x < E; x += 64) tab[x] = n_tok;
    asm volatile("" ::: "memory");
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      if (valid(id[q])) atomicMin(&tab[id[q]], lane + 64 * q);
    asm volatile("" ::: "memory");
    uint64_t F[4];
    int cF[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      F[q] = q < NQ ? ballot(valid(id[q]) && tab[id[q]] == lane + 64 * q) : 0ull;
      cF[q] = __popcll(F[q]);
    }
    // the item-th first-occurrence slot, and its expert
    int p = 0, qs = -1, ks = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (qs < 0 && item < p + cF[q]) qs = q, ks = item - p;
      p += cF[q];
    }
    if (qs < 0) return;  // past the routed experts (uniform)
    uint64_t Fs = F[0];
    int vs = id[0];
#pragma unroll
    for (int q = 1; q < 4; ++q)
      if (qs == q) Fs = F[q], vs = id[q];
    e = __builtin_amdgcn_readfirstlane(__shfl(vs, nth_set_bit(Fs, ks), 64));
  }
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
//
// `bid` is the workgroup's index in the launch's GEMV range (its block index
// in a GEMV-only launch) and `lds` the workgroup's dynamic LDS.
template <int MODE, int RPL, int PF_, int TC, int WAVES, int NIT, bool ROUTE, int UPW, int LPR>
__device__ __forceinline__ void gemv_item(const GemvLaunch a, int bid, u32x4_t* lds) {
  static_assert(UPW == 1 || (NIT > 0 && NIT % PF_ == 0), "units per workgroup need unrolled steps");
  static_assert(LPR == 8 || LPR == 16 || LPR == 32, "lanes per row");
  constexpr int NR = MODE == 0 ? 2 * RPL : RPL;  // weight rows per lane
  constexpr int NT = 64 * WAVES;
  constexpr int RG = 64 / LPR;                   // row groups per wave

  const int rows_per_wave = RG * RPL;
  const int chunks = a.n_out / rows_per_wave;           // row chunks (one wave each)
  const int slabs = (chunks + WAVES - 1) / WAVES;       // slabs of WAVES chunks
  const int groups = (slabs + UPW - 1) / UPW;           // workgroups per item
  const int item = (int)((unsigned)bid / (unsigned)groups);
  const int slab0 = (bid - item * groups) * UPW; // first of UPW slabs (units)
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

  // The one-token launches (one row per pass, 32 lanes per weight row: every
  // workgroup starts at once and each waits on the routing, then on its
  // first weights) raise the issue priority until the staged rows are in
  // place: M=1 16.20 -> 15.97 us per call.  The same made M=2 (two rows per
  // pass) and M=16 (8-lane rows) slower: 26.37 -> 26.84, 122.6 -> 123.9 us.
  constexpr bool kProloguePrio = LPR == 32 && TC == 1;
  if constexpr (kProloguePrio) __builtin_amdgcn_s_setprio(1);
  int e, T, f_lane = 0;
  int fl[4];
  if constexpr (ROUTE) {
    int dropped;
    // this wave's routing table, past the staged rows (gemv_route_lds_bytes)
    int* tab = reinterpret_cast<int*>(xc + TC * xc_pitch) + wid * a.num_experts;
    if (MODE == 1 && a.route_items) {
      if (a.n_tok <= 64)
        route_wave<1, false, true>(a, item, e, T, fl, dropped, tab);
      else
        route_wave<4, false, true>(a, item, e, T, fl, dropped, tab);
    } else if (a.n_tok <= 64) {
      route_wave<1, MODE == 0, false>(a, item, e, T, fl, dropped, tab);
    } else {
      route_wave<4, MODE == 0, false>(a, item, e, T, fl, dropped, tab);
    }
    if (MODE == 0 && bid == 0 && tid == 0) a.dropped_out[0] = dropped;
    // w13 leaves every item's expert (-1: no work) for the w2 launch
    if (MODE == 0 && a.route_items && slab0 == 0 && tid == 0) a.route_items[item] = e;
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
    // w13's four-row passes keep one step less in flight: the registers pay
    // for loading each activation row's pieces together (below).
    constexpr bool kRowBatch = MODE == 0 && NTOK == 4 && NIT > 0 && PF_ > 3 && NIT % 3 == 0;
    constexpr int PF = kRowBatch ? 3 : PF_;
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
      // Non-temporal weight loads: every 128-byte line is read whole by one
      // instruction (8 lanes of a row) and never again in the call, so it
      // need not displace cached lines (M=16 120.5 -> 109.6 us per call,
      // M=1 15.86 -> 15.13).  The scales' lines are read in pieces over 8
      // steps and keep the default policy.
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        wq[j] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t*>(wexp + (woff[j] + dw + gi * 16u)));
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

      // Passes of at most three rows (any pass of w2's short rows) load their
      // activation rows into registers ahead of the weights: loads return in
      // order, so a row load issued behind the weight prefetch would make the
      // staging below wait for the weights too, and the staging work and
      // barrier would follow their latency instead of running under it.
      // (w13's four-row passes have no registers to spare for it.)
      constexpr bool kEarly = NIT > 0 && (NTOK <= 3 || MODE == 1);
      constexpr int kOctMax = NIT * LPR * 4 + 4;  // row octets + the zero group
      constexpr int kStageIt = kEarly ? (kOctMax + NT - 1) / NT : 1;
      const int n_oct = kdim >> 3;
      u32x4_t xs[kEarly ? NTOK : 1][kStageIt];
      if constexpr (kEarly) {
#pragma unroll
        for (int t = 0; t < NTOK; ++t) {
          const int f = slot_of(min(t0 + t, T - 1));
          const int64_t arow = MODE == 0 ? f / a.topk : f;
          const u32x4_t* s4 = reinterpret_cast<const u32x4_t*>(a.act + arow * a.ld_act);
#pragma unroll
          for (int i = 0; i < kStageIt; ++i) {
            const int u = i * NT + tid;
            xs[t][i] = u32x4_t{0u, 0u, 0u, 0u};
            if (t < tc && u < n_oct) xs[t][i] = s4[u];
          }
        }
      }

#pragma unroll
      for (int p = 0; p < PF; ++p)
        if (NIT == 0 || p < UPW * NIT) {
          constexpr int kN = NIT > 0 ? NIT : 1;
          load_step(wb[p], sb[p], NIT ? p / kN : 0, NIT ? p % kN : min(p, n_it - 1));
        }

      // Stage this pass's activation rows (the whole workgroup).
      __syncthreads();
      if constexpr (kEarly) {
#pragma unroll
        for (int t = 0; t < NTOK; ++t)
          if (t < tc) {
#pragma unroll
            for (int i = 0; i < kStageIt; ++i)
              if (i * NT < n_oct + 4)
                stage_octet(xs[t][i], i * NT + tid, n_oct, xp + t * row_oct,
                            xc + t * xc_pitch, tid);
          }
      } else if constexpr (kRowBatch) {
        // A row's pieces are loaded together: one round trip per row instead
        // of one per piece.
        constexpr int kRowIt = (kOctMax + NT - 1) / NT;
        for (int t = 0; t < tc; ++t) {
          const int f = slot_of(t0 + t);
          const int64_t arow = MODE == 0 ? f / a.topk : f;
          const u32x4_t* s4 = reinterpret_cast<const u32x4_t*>(a.act + arow * a.ld_act);
          u32x4_t xr[kRowIt];
#pragma unroll
          for (int i = 0; i < kRowIt; ++i) {
            const int u = i * NT + tid;
            xr[i] = u32x4_t{0u, 0u, 0u, 0u};
            if (u < n_oct) xr[i] = s4[u];
          }
#pragma unroll
          for (int i = 0; i < kRowIt; ++i)
            if (i * NT < n_oct + 4)
              stage_octet(xr[i], i * NT + tid, n_oct, xp + t * row_oct, xc + t * xc_pitch, tid);
        }
      } else {
        for (int t = 0; t < tc; ++t) {
          const int f = slot_of(t0 + t);
          const int64_t arow = MODE == 0 ? f / a.topk : f;
          stage_row<NT>(a.act + arow * a.ld_act, kdim, xp + t * row_oct, xc + t * xc_pitch,
                        tid);
        }
      }
      __syncthreads();
      if constexpr (kProloguePrio) __builtin_amdgcn_s_setprio(0);

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


// ---- launch choices (host) ------------------------------------------------

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

// LDS of a self-routing launch: the staged rows, then each wave's routing
// table (one int per expert).
size_t gemv_route_lds_bytes(int tc, int kdim, int num_experts) {
  return gemv_lds_bytes(tc, kdim) + (size_t)kGemvWaves * (size_t)num_experts * sizeof(int);
}

// Launch shapes: output rows per lane (RPL) and prefetch depth (PF) of the
// two GEMVs, waves per workgroup.  w2's passes of four token rows have their
// own shape (_T4): 4 rows per lane with 2 steps in flight moves the same
// weight bytes per lane as 2 rows with 4 steps, in half the workgroups, and
// measured faster there (skewed M=64 133.6 -> 131.7 us, uniform M=32 203.1
// -> 198.7 us per call) but slower for passes of one or two rows.
// Overridable at build time for tuning sweeps.
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
#define W4A16_W2_PF 4
#endif
#ifndef W4A16_W13_RPL_T4
#define W4A16_W13_RPL_T4 W4A16_W13_RPL
#endif
#ifndef W4A16_W13_PF_T4
#define W4A16_W13_PF_T4 W4A16_W13_PF
#endif
#ifndef W4A16_W2_RPL_T4
#define W4A16_W2_RPL_T4 4
#endif
#ifndef W4A16_W2_PF_T4
#define W4A16_W2_PF_T4 2
#endif

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
  auto lds = [&](int t) {
    return a.ids ? gemv_route_lds_bytes(t, a.kdim, num_experts) : gemv_lds_bytes(t, a.kdim);
  };
  while (tc > 1 && lds(tc) > kMaxLds) tc >>= 1;
  return tc;
}

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

}  // namespace gemv_dev
}  // namespace
}  // namespace w4a16
