// Grouped dequant-GEMM on bf16 MFMA for experts with many tokens: the work
// items (device code shared by the MFMA-only launches and the mixed GEMV +
// MFMA launches).
//
// Reference kernels: _w4a16_moe_w1_fused_kernel (kernels/w4a16_moe.py:374-499)
// and _w4a16_moe_w2_kernel (:502-634): per 16-token block x 64-column tile,
// tl.dot of bf16 activations with bf16(dequantized weights), fp32 accumulate.
//
// Here one workgroup (8 waves, two per SIMD) owns one tile of one expert --
// up to 192 of its sorted (token, slot) pairs -- and one or more row tiles of
// 256 weight rows, run in turn.  The align kernel cuts an expert into as few
// such tiles as possible (one when it has at most 192 pairs), so every weight
// is dequantized once per expert at the prefill sizes and the dequantization
// work per MFMA falls as the expert's pair count grows.
//
//   * Every global load of the main loop is an LDS DMA (global_load_lds):
//     the gathered activation rows of a double step (64 elements, 128 bytes
//     per row), each wave's packed weights (32 rows x 32 bytes) and its
//     scales, three double steps ahead, so no vector register waits on
//     memory.  The waits are explicit vector-memory counts.
//   * A packed word becomes 8 bf16 weights bf16((c - 8) * s) with 17 VALU
//     instructions: two nibbles at a time are or-ed into fp16 numbers 1024 + c
//     (bits 0-3) or 1024 + 16 c (bits 4-7), and v_fma_mix_f32 turns each into
//     (c - 8) * s exactly, (1024 + c) * s - 1032 s or (1024 + 16 c) * (s / 16)
//     - 72 s; one v_cvt_pk_bf16_f32 rounds two of them.  The product before
//     the rounding is exact, so the bf16 weight is the reference's.
//   * MFMA v_mfma_f32_32x32x16_bf16 with the weights as the A operand and the
//     activations as B: the accumulator of a lane holds one token slot and 16
//     output rows in runs of 4, so the epilogue stores 4 neighbouring outputs
//     at a time.  A wave owns one 32-row block and up to 6 token blocks of 32
//     (6 x 16 fp32 accumulators).
//
// w13 (MODE 0): each wave's 32 rows are 16 gate rows and the matching 16 up
// rows, so each lane holds gate and up of the same output and the epilogue
// writes bf16(SiLU(gate) * up) -- the reference's rounding point.
// w2 (MODE 1): the epilogue multiplies by the routing weight and writes the
// partial row of the (token, slot) pair, rounded to bf16 like the reference's
// partial buffer (kernels/w4a16_moe.py:311) unless the call keeps fp32
// partials (M <= 4, where the reference accumulates in fp32).
//
// Workgroup ids are mapped so that the work items of one tile run on one XCD
// (consecutive hardware ids round-robin over the 8 XCDs) and share its L2 for
// the gathered activation rows, and each XCD runs its tallest tiles first.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace w4a16 {
namespace {
namespace mfma_dev {


typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// Native vectors: whole-value copies of HIP's union-based 4-vector structs
// end up in scratch memory instead of registers.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTN = kMfmaTileN;              // weight rows per tile (8 waves x 32)
constexpr int kTMMax = kMfmaTileMMax;        // token slots per tile, at most (6 blocks of 32)
constexpr int kAbufs = 4;                    // activation buffers (double steps in LDS)
constexpr int kDA = kAbufs - 1;              // activation DMAs run this many steps ahead
constexpr int kXcds = 8;
constexpr int kStepK = 64;                   // reduction elements per double step
constexpr int kUnroll = 4;                   // double steps per loop iteration
// MFMAs of a double step's last k-step issued before the end-of-step wait and
// barrier (the rest follow the next step's operand reads); -1: half of them.
// Overridable at build time for tuning sweeps.
#ifndef W4A16_MFMA_KSPLIT
#define W4A16_MFMA_KSPLIT -1
#endif
constexpr int kMfmaSplit = W4A16_MFMA_KSPLIT;
// Raw buffer resource word 3 (gfx9: no format, no swizzle) and a byte offset
// past any buffer's end (a store there is dropped, a load returns zeros).
constexpr int kRawBufferWord3 = 0x00020000;
constexpr uint32_t kDropOffset = 0xFFFFFFF0u;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Scale constants of one (row, group): codes at bits 0-3 of an fp16 half use
// (s, -1032 s), codes at bits 4-7 use (s / 16, -72 s).  Every product and
// addend is exact in fp32 for scales below 2^118.
struct GroupScale {
  float s0, b0, s1, b1;
};

__device__ __forceinline__ GroupScale group_scale(float s) {
  return GroupScale{s, -1032.0f * s, 0.0625f * s, -72.0f * s};
}

__device__ __forceinline__ float fma_half(uint32_t h2, int hi, float s, float b) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, h2);
  return fmaf((float)h[hi], s, b);
}

// SiLU with the hardware reciprocal (1 ulp), well inside the bf16 rounding
// that follows.
__device__ __forceinline__ float silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// s_waitcnt with only the vector-memory count: wait until at most n vector
// memory instructions of this wave are in flight (expcnt and lgkmcnt at their
// maxima, i.e. not waited for).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt lgkmcnt(N): at most N LDS instructions of this wave in flight.
// The LDS DMAs count in the vector-memory counter only, so the LDS reads of
// a wave complete in order and N counts the youngest reads exactly.
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4) | (N << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { wait_lgkmcnt<0>(); }

// Workgroup barrier without a memory fence: the activation tiles arrive by
// LDS DMA, which the vector-memory counter tracks, so a fence would wait for
// every load in flight (the weight prefetches too).  Each wave waits for its
// own DMA with wait_vmcnt first; the memory clobber keeps the compiler from
// moving LDS accesses across.
__device__ __forceinline__ void tile_barrier() { asm volatile("s_barrier" ::: "memory"); }

// A value the compiler cannot see through, in a vector register: the masks
// of the dequantization then stay operands of one v_and_or_b32.
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t v) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(v));
  return r;
}

struct Masks {
  uint32_t lo, hi, magic;
};

// 8 codes of one packed word (code i in bits 4i) -> 8 bf16 (code - 8) * s in
// code order.
__device__ __forceinline__ bf16x8_t dequant_word(uint32_t w, const GroupScale& g,
                                                 const Masks& mk) {
  const uint32_t w8 = w >> 8;
  const uint32_t p0 = (w & mk.lo) | mk.magic;   // codes 0, 4
  const uint32_t p1 = (w & mk.hi) | mk.magic;   // codes 1, 5 (times 16)
  const uint32_t p2 = (w8 & mk.lo) | mk.magic;  // codes 2, 6
  const uint32_t p3 = (w8 & mk.hi) | mk.magic;  // codes 3, 7 (times 16)
  const float v0 = fma_half(p0, 0, g.s0, g.b0);
  const float v1 = fma_half(p1, 0, g.s1, g.b1);
  const float v2 = fma_half(p2, 0, g.s0, g.b0);
  const float v3 = fma_half(p3, 0, g.s1, g.b1);
  const float v4 = fma_half(p0, 1, g.s0, g.b0);
  const float v5 = fma_half(p1, 1, g.s1, g.b1);
  const float v6 = fma_half(p2, 1, g.s0, g.b0);
  const float v7 = fma_half(p3, 1, g.s1, g.b1);
  const u32x4_t o = {pack_bf16x2(v0, v1), pack_bf16x2(v2, v3), pack_bf16x2(v4, v5),
                     pack_bf16x2(v6, v7)};
  return __builtin_bit_cast(bf16x8_t, o);
}

// LDS DMA of 16 or 4 bytes per lane: lane l's bytes at global base + voff
// land at LDS address lds + l * size (a wave-uniform LDS address, in M0).
// Written as inline assembly so that the compiler's memory counters see no
// LDS DMA: with one in sight it counts LDS reads out of order and waits for
// all of them (lgkmcnt(0)) wherever it needs one.  The waits for the DMAs
// themselves are explicit (wait_vmcnt); the memory clobber keeps LDS accesses
// in program order around them, and no other code here uses M0.  M0 must be
// written one wait state before the DMA.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(base), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
// The same 16-byte LDS DMA from a raw buffer: a lane whose offset is past the
// buffer's end writes zeros.
__device__ __forceinline__ void lds_dma16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff,
                                              uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void lds_dma4(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(voff), "s"(base), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>(p);
}

// Workgroup shapes.  NW waves (two per SIMD) of which wave w owns the
// 32-row MFMA block w of a row tile of 32 NW weight rows, and tiles of at
// most MCMAX token blocks of 32 slots:
//   * NW = 8, MCMAX = 6: 256 rows x 192 slots, one workgroup per CU (144 KB of
//     LDS), for the experts of large batches;
//   * NW = 4, MCMAX = 2: 128 rows x 64 slots, two workgroups per CU (58 KB
//     each), for tiles of at most 64 slots: with few pairs per expert a
//     launch is latency-bound, and a second workgroup on the CU runs while
//     the other waits at its barrier or on its loads, and twice as many work
//     items spread over the CUs.
// LDS of one workgroup (all three rings are filled by LDS DMA):
//   A  kAbufs buffers of 32 MCMAX rows x 128 bytes: the gathered activation
//      rows of one double step.  Chunk c (16 bytes) of row r sits at
//      r * 128 + 16 * (c ^ g(r)), g(r) = (r ^ (r / 8)) % 8, so the lanes
//      reading one chunk of 8 (or 16) neighbouring rows hit 8 (16) different
//      16-byte bank groups of a 128-byte (256-byte) bank row.
//   W  WSLOTS slots x NW waves x 2 KB: a wave's packed weights of a pair of
//      double steps (64 bytes of each of its 32 rows), as two DMAs of 16
//      rows: DMA h, lane l holds row r = 16 h + l / 4, bytes 16 c of the
//      pair's 64, c = (l % 4) ^ ((r % 16) / 4), at h * 1024 + l * 16 (the
//      swizzle spreads a read of 16 rows over all banks).  The weights run 2 WSLOTS - 1 double
//      steps ahead, deeper than the activations: they come from HBM, the
//      activation rows mostly from L2.
//   S  2 slots x NW waves x 512 B: a wave's scales of one loop iteration (8
//      groups of 32 elements), lane j's bytes (lanes 0-31) at j times the
//      DMA size.
template <int NW, int MCMAX, int WSLOTS>
struct TileGeo {
  static constexpr int kWaves = NW;
  static constexpr int kMcMax = MCMAX;
  static constexpr int kWslots = WSLOTS;
  static constexpr int kDW = 2 * WSLOTS - 1;     // weight DMAs run this many steps ahead
  static constexpr int kTN = 32 * NW;            // weight rows of a row tile
  static constexpr int kTM = 32 * MCMAX;         // token slots of a tile, at most
  static constexpr int kAbuf = kTM * 128;        // one activation buffer
  static constexpr int kWslot = NW * 2048;
  static constexpr int kSslot = NW * 512;
  static constexpr int kOffW = kAbufs * kAbuf;
  static constexpr int kOffS = kOffW + kWslots * kWslot;
  static constexpr int kLdsTotal = kOffS + 2 * kSslot;
  static constexpr int kWgsPerCu = NW == 8 ? 1 : 2;
  static_assert(kTM <= kTMMax, "tile height");
  static_assert((kLdsTotal + kTM * 8) * kWgsPerCu <= 160 * 1024, "LDS of the workgroups of a CU");
};
#ifndef W4A16_MFMA_WSLOTS_BIG
#define W4A16_MFMA_WSLOTS_BIG 2
#endif
#ifndef W4A16_MFMA_WSLOTS_SMALL
#define W4A16_MFMA_WSLOTS_SMALL 2
#endif
using BigTile = TileGeo<8, 6, W4A16_MFMA_WSLOTS_BIG>;
using SmallTile = TileGeo<4, 2, W4A16_MFMA_WSLOTS_SMALL>;

// LDS DMAs a wave issues after the last one that double step t + 1 needs,
// counted to the end of step t's issues.  Step s issues, in this order: the
// scales of iteration s / 4 + 1 (s % 4 == 0, s >= 0; the prologue issues
// those of iteration 0 first of all), NA activation DMAs for step s + kDA
// (when s + kDA >= 0), and for odd s the two weight DMAs of the pair of
// steps s + DW, s + DW + 1 (when s + DW >= 0); the prologue issues steps
// -DW .. -1 the same way.  Step t + 1 needs its activations, its weight pair
// and its iteration's scales, so the wait before it is vmcnt(dmas_behind(t)).
constexpr int dmas_behind(int t, int NA, int DW, int KS) {
  const int u = t + 1;
  // its activations (step, position; a wave with NA = 0 issues none), then
  // its weight pair, position 2, and its scales, position 0
  int bs = NA > 0 ? u - kDA : -1000, bp = 1;
  const int ws = 2 * (u / 2) - DW;
  if (ws >= bs) bs = ws, bp = 2;
  if (u >= 4) {
    const int ss = 4 * (u / 4) - 4;
    if (ss > bs) bs = ss, bp = 0;
  }
  auto acts = [&](int st) { return st + kDA >= 0 ? NA : 0; };
  auto wts = [&](int st) { return ((st & 1) && st + DW >= 0) ? 2 : 0; };
  int n = (bp == 0 ? acts(bs) : 0) + (bp <= 1 ? wts(bs) : 0);
  for (int st = bs + 1; st <= t; ++st) n += (st >= 0 && st % 4 == 0 ? KS : 0) + acts(st) + wts(st);
  return n;
}
// The loop waits with the count of a step far from the start, for every
// step with the same t % 4: safe when no earlier step has fewer DMAs behind
// its needed ones (the prologue's pseudo-steps issue fewer).
constexpr bool steady_wait_safe(int NA, int DW, int KS) {
  for (int t = 0; t < 32; ++t)
    if (dmas_behind(t, NA, DW, KS) < dmas_behind(16 + t % 4, NA, DW, KS)) return false;
  return true;
}
static_assert(BigTile::kTN == kTN, "row tile of the big tiles");
static_assert(SmallTile::kTM == kMfmaTileMSmall, "small tiles are the 64-slot tiles");
static_assert(SmallTile::kTN == kMfmaTileNSmall, "row tile of the small tiles");

// One tile of MC token blocks (32 slots each).  GSHIFT = log2(group / 32).
//
// Wave w owns one 32-row MFMA block of the row tile's 32 NW weight rows: for
// w13 rows 0-15 of the block are gate rows and rows 16-31 the matching up
// rows (output columns 16 w ..), so accumulator registers r and r + 8 of a
// lane hold gate and up of one output; for w2 rows 32 w ...  Two waves share
// each SIMD: one issues MFMAs while the other waits on LDS or dequantizes.
//
// Every global load of the main loop is an LDS DMA, issued about three
// double steps ahead, so no vector register waits on memory there.  The
// weights go by pairs of double steps: 64 contiguous bytes of a row per DMA
// lane group, half the cache-line requests of per-step 32-byte pieces.
// Issue order per double step t (fixed by scheduling barriers; the prologue
// issues pseudo-steps -3 .. -1 the same way): [the next iteration's scales
// when t % 4 == 0] [NA activation DMAs of step t + 3] [when t is odd: the 2
// weight DMAs of pair (t + 3) / 2, i.e. steps t + 3 and t + 4, into the slot
// of t's own pair, whose words the wave has read into registers during step
// t - 1].  In k-step 3 of step t each wave waits until the last of the DMAs
// step t + 1 needs has landed -- the vector-memory count of the instructions
// behind it is exact below -- and the workgroup barrier then makes every
// wave's activation rows visible.
template <int MODE, int GSHIFT, int MC, int NA, class G>
__device__ __forceinline__ void run_tile(const MfmaLaunch& a, int e, int nt0, int nrt,
                                         const int* s_f, const float* s_wt,
                                         unsigned char* lds) {
  constexpr int kWaves = G::kWaves;
  constexpr int kTileN = G::kTN;
  constexpr int kAbufG = G::kAbuf;
  constexpr int kWslot = G::kWslot;
  static_assert(MC >= 1 && MC <= G::kMcMax, "token blocks of a tile");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int j = lane & 31;
  const int q = lane >> 5;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  const int kdim = a.kdim;
  const int T = kdim / kStepK;  // double steps of one row tile, a multiple of kUnroll
  const int IT = T / kUnroll;    // loop iterations of one row tile
  const int GT = nrt * T;        // double steps of the item (nrt row tiles)
  const int gpr = kdim / a.group;
  // Row tile and local step of global double step gs (clamped to the item's
  // last, GT - 1), from the row tile rt_cur of the current step: the DMAs
  // run at most DW steps ahead, at most two row tiles past rt_cur (T >= 4,
  // DW < 2 T, checked by the launcher).
  auto split_step = [&](int gs, int rt_cur, int& rt, int& k) {
    const int gc = min(gs, GT - 1);
    rt = rt_cur + (gc >= (rt_cur + 1) * T) + (gc >= (rt_cur + 2) * T);
    k = gc - rt * T;
  };
  constexpr int kWslotsG = G::kWslots;
  constexpr int DW = G::kDW;
  static_assert(steady_wait_safe(NA, DW, GSHIFT == 1 ? 2 : 1), "DMA wait counts");
  static_assert(dmas_behind(17, NA, DW, GSHIFT == 1 ? 2 : 1) + MC * 2 < 64, "vmcnt range");
  static_assert(dmas_behind(19, NA, DW, GSHIFT == 1 ? 2 : 1) < 64, "vmcnt range");
  // Slot of weight pair p, from the slot of pair 2 it (wave-uniform).
  auto wslot = [](int base, int c) {
    int v = base + c;
    while (v >= kWslotsG) v -= kWslotsG;
    return v;
  };

  // ---- activation DMA: the tile's 4 MC DMAs of 1 KB (8 rows each) are dealt
  // round robin over the waves, so wave w issues NA = ceil((4 MC - w) / NW)
  // of them (the caller instantiates both counts of an uneven share); DMA k
  // fills rows 8 k .. 8 k + 7 of the buffer: lane l writes row r = 8 k + l / 8
  // at chunk position l % 8, so it fetches chunk (l % 8) ^ g(r) of that row.
  // Lanes of padding slots read past the end of the activation buffer, so
  // their rows are zeros: the MFMAs over them compute what they would with
  // any row (their outputs are not stored) and draw less power.
  static_assert(NA >= 0 && NA <= (4 * MC + kWaves - 1) / kWaves, "activation DMAs per wave");
  constexpr int kNA1 = NA > 0 ? NA : 1;
  uint32_t a_off[kNA1];  // byte offset of this lane's source row + chunk
  int a_dst[kNA1];       // LDS byte offset within a buffer
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int k = kWaves * i + wid;  // < 4 MC for this wave's NA
    a_dst[i] = k * 1024;
    const int r = 8 * k + (lane >> 3);
    const int f = s_f[r];
    const uint32_t row = MODE == 0 ? (uint32_t)(f / a.topk) : (uint32_t)f;
    const int g = (lane >> 3) ^ (k & 7);  // swizzle of row r (see above)
    a_off[i] = f < a.n_tok ? row * (uint32_t)a.ld_act * 2u + (uint32_t)(((lane & 7) ^ g) * 16)
                           : kDropOffset;
  }
  const char* const act = reinterpret_cast<const char*>(a.act);
  const uint32_t act_bytes = __builtin_amdgcn_readfirstlane(
      (uint32_t)(MODE == 0 ? a.n_tok / a.topk : a.n_tok) * (uint32_t)a.ld_act * 2u);
  // The item's row tiles share the activation rows: local step k of any.  The
  // step's column offset moves the buffer's base, so that the padding lanes'
  // offset stays past the end; a live lane's bytes end within row f, before
  // act_bytes.
  auto dma_a1 = [&](int k, int buf, int i) {
    const uint32_t koff = __builtin_amdgcn_readfirstlane((uint32_t)k * (kStepK * 2));
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(act + koff), 0, act_bytes, kRawBufferWord3);
    lds_dma16_buf(rsrc, a_off[i], lds_addr(lds + buf * kAbufG + a_dst[i]));
  };
  auto dma_a = [&](int k, int buf) {
#pragma unroll
    for (int i = 0; i < NA; ++i) dma_a1(k, buf, i);
  };
  // Read addresses: row 32 m + j, chunk 4 q + u -> position (4 q + u) ^ g,
  // g = (j % 8) ^ (j / 8) ^ 4 (m % 2); row 32 (m % 2) + j is in a_rd, the
  // m / 2 part is an immediate offset.
  uint32_t a_rd[2][4];
#pragma unroll
  for (int par = 0; par < 2; ++par)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      a_rd[par][u] = (uint32_t)((32 * par + j) * 128 +
                                16 * ((4 * q + u) ^ (j & 7) ^ (j >> 3) ^ (4 * par)));

  // ---- the weight row of this lane ------------------------------------------
  // Row tile nt0 + rt moves every row by kTileN / 2 (w13: gate and up) or
  // kTileN.
  constexpr int kRowsPerTile = MODE == 0 ? kTileN / 2 : kTileN;
  // Weight row of local row r (0..31) of the wave's block.
  auto wrow = [&](int r) {
    if (MODE == 0) {
      const int col = nt0 * (kTileN / 2) + 16 * wid + (r & 15);
      return r < 16 ? col : a.n_out + col;  // gate, or the matching up row
    } else {
      return nt0 * kTileN + 32 * wid + r;
    }
  };
  const int grow = wrow(j);
  const int64_t e_rows = (int64_t)e * rows_total;
  const char* const wexp = reinterpret_cast<const char*>(a.w) + e_rows * (kdim / 2);
  const char* const sexp = reinterpret_cast<const char*>(a.s) + e_rows * gpr * 2;
  // Weight DMA h of a pair: lane l lands at LDS position l (16 bytes each) of
  // the DMA's kilobyte: row r = 16 h + l / 4, slot l % 4 of the row's 64
  // bytes, which holds the row's 16-byte group (l % 4) ^ sw(r % 16),
  // sw(r) = (r / 4) % 4.  The reads below take one group of 16 rows at once,
  // 64 bytes apart: without the swizzle four of those rows share every bank
  // (LDS banks repeat every 256 bytes).
  auto wswz = [](int r) { return (r >> 2) & 3; };
  uint32_t w_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    w_off[h] = (uint32_t)wrow(16 * h + (lane >> 2)) * (uint32_t)(kdim / 2) +
               16u * (uint32_t)((lane & 3) ^ wswz(lane >> 2));
  // Lane (j, q) reads 16-byte group 2 (t % 2) + q of row j's pair block, at
  // slot group ^ sw(j % 16): w_rd[t % 2].
  uint32_t w_rd[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
    w_rd[b] = (uint32_t)((j >> 4) * 1024 + (j & 15) * 64 + 16 * ((2 * b + q) ^ wswz(j & 15)));
  const uint32_t s_off = (uint32_t)grow * (uint32_t)gpr * 2u;
  unsigned char* const w_lds = lds + G::kOffW + wid * 2048;  // + slot * kWslot
  unsigned char* const s_lds = lds + G::kOffS + wid * 512;   // + slot * kSslot
  const uint32_t w_tile = (uint32_t)kRowsPerTile * (uint32_t)(kdim / 2);
  const uint32_t s_tile = (uint32_t)kRowsPerTile * (uint32_t)gpr * 2u;
  // The pair of double steps k, k + 1 (k even) of row tile rt.
  auto dma_w = [&](int rt, int k, int slot) {
    const uint32_t koff = (uint32_t)rt * w_tile + (uint32_t)(k >> 1) * 64u;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      lds_dma16(wexp, w_off[h] + koff, lds_addr(w_lds + slot * kWslot + h * 1024));
  };
  // Scales of one loop iteration (8 groups of 32 elements): 16, 8 or 4 bytes
  // of the row by group size, naturally aligned (kdim % 256 == 0), as one
  // 16-byte DMA, two 4-byte DMAs or one 4-byte DMA, by the lanes q = 0 (the
  // lanes q = 1 of the same rows read them from there).
  constexpr int kSBytes = GSHIFT == 0 ? 16 : 4;
  constexpr int kSDmas = GSHIFT == 1 ? 2 : 1;
  // Scales of global iteration git (clamped to the item's last).
  auto dma_s = [&](int git, int slot) {
    const int gc = min(git, nrt * IT - 1);
    const int rt = gc / IT;  // once per iteration
    const uint32_t i = (uint32_t)(gc - rt * IT);
    if (q == 0) {
#pragma unroll
      for (int d = 0; d < kSDmas; ++d) {
        const uint32_t voff = s_off + (uint32_t)rt * s_tile + i * (16u >> GSHIFT) + 4u * d;
        const uint32_t dst = lds_addr(s_lds + slot * G::kSslot + d * 256);
        if constexpr (GSHIFT == 0)
          lds_dma16(sexp, voff, dst);
        else
          lds_dma4(sexp, voff, dst);
      }
    }
  };
  // The scale word (2 bf16) holding group 2 tp + q (in units of 32
  // elements) of the iteration, and its bf16 half.
  auto scale_word = [&](int slot, int tp) {
    const unsigned char* p = s_lds + slot * G::kSslot + j * kSBytes;
    if constexpr (GSHIFT == 0) return *reinterpret_cast<const uint32_t*>(p + 4 * tp);
    else if constexpr (GSHIFT == 1) return *reinterpret_cast<const uint32_t*>(p + 256 * (tp >> 1));
    else return *reinterpret_cast<const uint32_t*>(p);
  };
  auto scale_value = [&](uint32_t word, int tp) {
    const int half = GSHIFT == 0 ? q : GSHIFT == 1 ? (tp & 1) : (tp >> 1);
    const uint32_t bits = half ? (word & 0xFFFF0000u) : (word << 16);
    return __uint_as_float(bits);
  };

  const Masks mk{opaque_vgpr(0x000F000Fu), opaque_vgpr(0x00F000F0u), opaque_vgpr(0x64006400u)};

  f32x16_t acc[MC];
  auto clear_acc = [&]() {
#pragma unroll
    for (int m = 0; m < MC; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[m][r] = 0.0f;
  };
  clear_acc();

  // Operands of a double step that are ready before it starts: the packed
  // weight words and the scale of the lane's group (the wave's own DMAs, read
  // in k-step 3 of the previous step and turned into the group constants and
  // the k-step 0 weights there, before the barrier), and the activation
  // fragments of k-steps 0 and 1 (read behind the barrier).
  u32x4_t wq, wq_next;
  uint32_t sw_next;
  GroupScale gs;
  bf16x8_t af[4][MC], bw[2];  // af[u]: fragments of k-step u
  auto read_a = [&](const unsigned char* abuf, int u, bf16x8_t (&dst)[MC]) {
#pragma unroll
    for (int m = 0; m < MC; ++m)
      dst[m] = *reinterpret_cast<const bf16x8_t*>(abuf + a_rd[m & 1][u] + (m >> 1) * 2 * 32 * 128);
  };
  // The step's weight words (pair slot wsl) and scale word (this wave's own
  // DMAs).
  auto read_w_operands = [&](int tp, int wsl, int sslot) {
    wq_next = *reinterpret_cast<const u32x4_t*>(w_lds + wsl * kWslot + w_rd[tp & 1]);
    sw_next = scale_word(sslot, tp);
  };
  // Group constants and k-step 0 weights of the step whose words were read.
  auto start_step_weights = [&](int tp) {
    gs = group_scale(scale_value(sw_next, tp));
    bw[0] = dequant_word(wq_next[0], gs, mk);
    wq = wq_next;
  };
  // The step's k-step 0 and 1 activation fragments (into af[0], af[1]).
  auto read_step_acts = [&](int tp) {
    read_a(lds + tp * kAbufG, 0, af[0]);
    read_a(lds + tp * kAbufG, 1, af[1]);
  };

  // Output of row tile nt.  Accumulator register r of a 32x32 block holds
  // weight row 8 (r / 4) + 4 q + r % 4 of the wave's block and token slot j;
  // the slot's token row and routing weight (w2) are in LDS (s_f, s_wt).
  // The epilogue's stores: raw buffer stores over the output rows, issued by
  // every lane -- a slot past the tile's pairs stores at an offset past the
  // buffer's end, which the hardware drops -- so a row tile's epilogue issues
  // the same number of vector-memory instructions on every wave, at least
  // kEpiStores, and the workgroup's last wait leaves them in flight.  Lanes
  // q = 0 and q = 1 of slot j hold alternating runs of 4
  // outputs; v_permlane32_swap trades runs between the two halves of the
  // wave so that each lane stores 8 consecutive outputs (16 bytes) at once,
  // and for w2 v_permlane16_swap then trades pieces between slots j and
  // j + 16 so that each store instruction writes 16 slots x 64 bytes (the
  // wave's 32 rows of each) instead of 32 slots x 32 bytes: a quarter of the
  // store instructions and write requests of storing each run of 4 on its
  // own.
  constexpr int kEpiStores = MC * (MODE == 0 ? 1 : 2);
  const uint32_t out_elt = (MODE == 1 && !a.partial_bf16) ? 4u : 2u;
  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      a.out, 0, (uint32_t)a.n_tok * (uint32_t)a.n_out * out_elt, kRawBufferWord3);
  // swap_halves(a, b): the a of lanes 32-63 and the b of lanes 0-31 trade
  // places -- lanes 0-31 keep their a and get, as b, the a of lane + 32;
  // lanes 32-63 get, as a, the b of lane - 32 and keep their b.
  auto swap_halves = [](u32x2_t& a2, u32x2_t& b2) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const auto r = __builtin_amdgcn_permlane32_swap(a2[w], b2[w], false, false);
      a2[w] = r[0];
      b2[w] = r[1];
    }
  };
  // swap_rows16(a, b): the a of lane rows 1 and 3 (lanes 16-31, 48-63) and
  // the b of rows 0 and 2 trade places -- lanes of rows 0, 2 keep their a
  // and get, as b, the a of lane + 16; lanes of rows 1, 3 get, as a, the b
  // of lane - 16 and keep their b.
  auto swap_rows16 = [](u32x2_t& a2, u32x2_t& b2) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const auto r = __builtin_amdgcn_permlane16_swap(a2[w], b2[w], false, false);
      a2[w] = r[0];
      b2[w] = r[1];
    }
  };
  auto store16 = [&](const u32x2_t& lo, const u32x2_t& hi, uint32_t byte_off) {
    const u32x4_t v = {lo[0], lo[1], hi[0], hi[1]};
    __builtin_amdgcn_raw_buffer_store_b128(v, out_rsrc, byte_off, 0, 0);
  };
  auto write_out = [&](int nt) {
#pragma unroll
    for (int m = 0; m < MC; ++m) {
      const int f = s_f[32 * m + j];
      const bool live = f < a.n_tok;  // the same for both lanes of a slot
      if (MODE == 0) {
        // Lane (q, j): r < 8 gate column 8 (r / 4) + 4 q + r % 4 of the
        // wave's 16, r + 8 its up row; runs i4 = 0, 1 are columns 4 q + 0..3
        // and 8 + 4 q + 0..3.  After the swap lane q holds columns 8 q .. +7.
        u32x2_t hv[2];
#pragma unroll
        for (int i4 = 0; i4 < 2; ++i4) {
          float h[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) h[c] = silu(acc[m][4 * i4 + c]) * acc[m][8 + 4 * i4 + c];
          hv[i4] = u32x2_t{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
        }
        swap_halves(hv[0], hv[1]);
        const uint32_t e0 =
            (uint32_t)f * (uint32_t)a.n_out + nt * (kTileN / 2) + 16 * wid + 8 * q;
        store16(hv[0], hv[1], live ? e0 * 2u : kDropOffset);
      } else {
        // Lane (q, j): runs i4 = 0..3 are rows 8 i4 + 4 q + 0..3 of the
        // wave's 32 for slot j.  After the half swaps lane (q, j) holds rows
        // 8 q .. +7 (runs 0, 1) and 16 + 8 q .. +7 (runs 2, 3); after the row
        // swaps its first piece is rows 16 h + 8 q .. +7 of slot j % 16 and
        // its second the same rows of slot 16 + j % 16 (h = j / 16).
        const float wt = s_wt[32 * m + j];
        const uint32_t e0 = (uint32_t)f * (uint32_t)a.n_out + nt * kTileN + 32 * wid;
        if (a.partial_bf16) {
          u32x2_t pv[4];
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4)
            pv[i4] = u32x2_t{pack_bf16x2(acc[m][4 * i4 + 0] * wt, acc[m][4 * i4 + 1] * wt),
                             pack_bf16x2(acc[m][4 * i4 + 2] * wt, acc[m][4 * i4 + 3] * wt)};
          swap_halves(pv[0], pv[1]);
          swap_halves(pv[2], pv[3]);
          swap_rows16(pv[0], pv[2]);
          swap_rows16(pv[1], pv[3]);
          const int f1 = s_f[32 * m + (j & 15)], f2 = s_f[32 * m + (j | 16)];
          const uint32_t rows = nt * kTileN + 32 * wid + 16 * (j >> 4) + 8 * q;
          store16(pv[0], pv[1],
                  f1 < a.n_tok ? ((uint32_t)f1 * (uint32_t)a.n_out + rows) * 2u : kDropOffset);
          store16(pv[2], pv[3],
                  f2 < a.n_tok ? ((uint32_t)f2 * (uint32_t)a.n_out + rows) * 2u : kDropOffset);
        } else {
          // fp32 partials (few-token calls): 4 rows are already 16 bytes.
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            const f32x4_t v = {acc[m][4 * i4 + 0] * wt, acc[m][4 * i4 + 1] * wt,
                               acc[m][4 * i4 + 2] * wt, acc[m][4 * i4 + 3] * wt};
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4_t, v), out_rsrc,
                live ? (e0 + 8 * i4 + 4 * q) * 4u : kDropOffset, 0, 0);
          }
        }
      }
    }
  };
  // Prologue: the scales of iteration 0, then pseudo-steps -DW .. -1 (the
  // activation DMAs of steps 0 .. kDA - 1, the weight pairs of steps
  // 0 .. DW).
  dma_s(0, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = -DW; s < 0; ++s) {
    int rt, k;
    if (s + kDA >= 0) {
      split_step(s + kDA, 0, rt, k);
      dma_a(k, s + kDA);
    }
    __builtin_amdgcn_sched_barrier(0);
    if ((s & 1) && s + DW >= 0) {
      split_step(s + DW, 0, rt, k);
      dma_w(rt, k, ((s + DW) / 2) % kWslotsG);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vmcnt<dmas_behind(-1, NA, DW, kSDmas)>();
  read_w_operands(0, 0, 0);
  start_step_weights(0);
  tile_barrier();
  __builtin_amdgcn_sched_barrier(0);
  read_step_acts(0);

  // Global iterations over the item's row tiles; every IT of them finish a
  // row tile, whose outputs are written before the next one accumulates.
  // The DMA stream runs on across the row-tile boundary.
  const int n_it = nrt * IT;
  int rt_cur = 0;
  int ws0 = 0;  // slot of weight pair 2 it
  for (int it = 0; it < n_it; ++it) {
    // One double step; tp = t % 4 is a compile-time constant.
    auto step = [&](auto tp_c) {
      constexpr int tp = decltype(tp_c)::value;
      const int t = it * kUnroll + tp;
      int rt_a, k_a;  // row tile and local step of this step's activation DMAs
      split_step(t + kDA, rt_cur, rt_a, k_a);
      int rt_w = 0, k_w = 0;  // and of its weight pair (odd t)
      if (tp & 1) split_step(t + DW, rt_cur, rt_w, k_w);
      // This step's DMAs are spread over k-steps 0-2 so that the address
      // unit drains them behind the MFMAs: [scales when tp == 0] and
      // activation DMA 0 in k-step 0, activation DMA u in k-step u, the
      // weight DMAs (odd steps: pair (t + DW) / 2) in k-step 2 -- the order
      // dmas_behind counts.  Buffer (t + kDA) % kAbufs was read last for step
      // t - 1, before the barrier of step t - 1; the slot of pair
      // (t + DW) / 2 held the pair of steps t - 1 and t, whose words this
      // wave read during steps t - 2 and t - 1; scale slot (it + 1) % 2 was
      // read last for step 3 of iteration it - 1, during step 2.
      auto issue_dmas = [&](int u) {
        __builtin_amdgcn_sched_barrier(0);
        if (tp == 0 && u == 0) dma_s(it + 1, (it + 1) & 1);
#pragma unroll
        for (int i = 0; i < NA; ++i)
          if (i == u || (u == 2 && i > 2)) dma_a1(k_a, (tp + kDA) % kAbufs, i);
        if (u == 2 && (tp & 1)) dma_w(rt_w, k_w, wslot(ws0, (tp + DW) / 2));
        __builtin_amdgcn_sched_barrier(0);
      };

      const unsigned char* const acur = lds + tp * kAbufG;
      constexpr int tn = (tp + 1) & 3;
      auto mfmas = [&](int c, int m0, int m1) {
#pragma unroll
        for (int m = m0; m < m1; ++m)
          acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[c & 1], af[c][m], acc[m], 0, 0, 0);
      };
      // Software pipeline over the 4 MFMA k-steps u: the activation
      // fragments of u + 2 are read and the weights of u + 1 dequantized
      // while the MFMAs of u run; k-step u waits only for its own fragments
      // (the compiler's exact LDS counts keep the later reads in flight).
      // The wave raises its issue priority over these interleaved MFMA +
      // dequantization groups, so that the SIMD's other wave (reading
      // fragments, waiting or issuing DMAs) does not delay its MFMAs: M=4096
      // 960 -> 951 us, M=1024 469 -> 460 us per call; also raising it for
      // k-step 3's MFMAs before the barrier measured slower (963, 470).
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        issue_dmas(u);
        if (u < 2) read_a(acur, u + 2, af[u + 2]);
        __builtin_amdgcn_s_setprio(1);
        mfmas(u, 0, MC);
        bw[(u + 1) & 1] = dequant_word(wq[u + 1], gs, mk);
        // The fragments' LDS reads, then each MFMA followed by a share of
        // the next dequantization.
        if (u < 2) __builtin_amdgcn_sched_group_barrier(0x100, MC, 0);
#pragma unroll
        for (int i = 0; i < MC; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, (17 + MC - 1) / MC, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
      }
      // k-step 3: the wait for step t+1's data and the wave's reads of its
      // own weight words and scale of t+1; the first MFMAs with t+1's group
      // constants and k-step 0 weights computed between them; the barrier
      // (every wave's activation rows of t+1 have landed); t+1's activation
      // reads (into af[0], af[1]) behind the remaining MFMAs.
      __builtin_amdgcn_sched_barrier(0);
      // Step t+1's data (activations, weight pair, scales) has landed once
      // at most dmas_behind(t) of this wave's DMAs are in flight; the count
      // depends on t % 4 only.
      // (After a row tile's epilogue the first waits also wait for its
      // stores: counting them instead, measured, gained nothing on w2 and
      // cost w13 ~2 % through the loop's code.)
      wait_vmcnt<dmas_behind(4 * kUnroll + tp, NA, DW, kSDmas)>();
      read_w_operands(tn, wslot(ws0, (tp + 1) / 2), tp == 3 ? ((it + 1) & 1) : (it & 1));
      __builtin_amdgcn_sched_barrier(0);
      constexpr int kSplit = kMfmaSplit < 0 ? (MC + 1) / 2 : (kMfmaSplit > MC ? MC : kMfmaSplit);
      mfmas(3, 0, kSplit);
      start_step_weights(tn);
#pragma unroll
      for (int i = 0; i < kSplit; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, (23 + kSplit - 1) / (kSplit > 0 ? kSplit : 1), 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      tile_barrier();
      __builtin_amdgcn_sched_barrier(0);
      read_step_acts(tn);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(3, kSplit, MC);
    };
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
    if (it + 1 == (rt_cur + 1) * IT) {
      write_out(nt0 + rt_cur);
      clear_acc();
      ++rt_cur;
    }
    ws0 = wslot(ws0, 2);
  }
  // The reads of a step past the last (clamped DMAs, never used) are the
  // only LDS reads still in flight.
  wait_lgkmcnt0();
  // No LDS DMA may still be in flight when the workgroup's LDS is released:
  // every DMA was issued before the last epilogue's stores, which need not
  // land before the workgroup ends.
  wait_vmcnt<kEpiStores>();
}

// One work item of a launch: `bid` is the workgroup's index in the launch's
// MFMA range, which starts at block 0 (the XCD of a block is its index
// modulo 8), `lds` the workgroup's dynamic LDS (G::kLdsTotal bytes) and
// s_f / s_wt its G::kTM slots' pair indices and routing weights.
template <int MODE, int GSHIFT, class G>
__device__ __forceinline__ void mfma_item(const MfmaLaunch& a, int bid, unsigned char* lds,
                                          int* s_f, float* s_wt) {
  constexpr int kWaves = G::kWaves;

  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  const int n_tiles_n = rows_total / G::kTN;
  // A work item is up to row_tiles consecutive row tiles of one token tile.
  const int per_item = a.row_tiles;
  const int items_per_tile = (n_tiles_n + per_item - 1) / per_item;
  // Tiles are dealt over the 8 XCDs (consecutive workgroup ids go to
  // consecutive XCDs), in rounds of 8 that alternate direction, and the work
  // items of one tile run back to back on its XCD, sharing its L2 for the
  // gathered activation rows.  The align kernel lists the tiles tallest
  // first, so every XCD starts its longest tiles first and hands out the
  // rest as its CUs free up.  The grid is sized for the most tiles a routing
  // can produce; workgroups past the real count (header[2]) leave at once.
  const int xcd = bid % kXcds, slot = bid / kXcds;
  const int round = slot / items_per_tile;
  const int tile = kXcds * round + ((round & 1) ? kXcds - 1 - xcd : xcd);
  if (tile >= a.header[2]) return;
  const int nt0 = (slot - round * items_per_tile) * per_item;
  const int nrt = min(per_item, n_tiles_n - nt0);
  const int4 info = a.tiles[tile];
  const int e = info.x, start = info.y;
  const int count = min(info.z, G::kTM);

  for (int i = threadIdx.x; i < G::kTM; i += kWaves * 64) {
    const int f = i < count ? a.sorted[start + i] : a.n_tok;
    s_f[i] = f;
    s_wt[i] = (MODE == 1 && f < a.n_tok) ? a.topk_w[f] : 0.0f;
  }
  __syncthreads();

  // Wave w issues ceil((4 MC - w) / NW) activation DMAs per step: when NW
  // does not divide 4 MC, the first (4 MC) % NW waves one more than the others.
  const int wid = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
#define W4A16_MFMA_TILE(MC_)                                                             \
  case MC_:                                                                              \
    if constexpr (MC_ <= G::kMcMax) {                                                    \
      if (wid < (4 * MC_) % kWaves)                                                      \
        run_tile<MODE, GSHIFT, MC_, (4 * MC_ + kWaves - 1) / kWaves, G>(a, e, nt0, nrt,  \
                                                                       s_f, s_wt, lds);  \
      else                                                                               \
        run_tile<MODE, GSHIFT, MC_, (4 * MC_) / kWaves, G>(a, e, nt0, nrt, s_f, s_wt,    \
                                                           lds);                         \
    }                                                                                    \
    break;
  switch ((count + 31) >> 5) {
    W4A16_MFMA_TILE(1)
    W4A16_MFMA_TILE(2)
    W4A16_MFMA_TILE(3)
    W4A16_MFMA_TILE(4)
    W4A16_MFMA_TILE(5)
    W4A16_MFMA_TILE(6)
    default: break;
  }
#undef W4A16_MFMA_TILE
}


// Whether launch `a` suits the work items of geometry G: whole row tiles,
// whole loop iterations, a tile height G holds, 16-byte aligned scales, the
// 32-bit activation offsets, and DMAs that run at most two row tiles ahead.
template <int MODE, class G>
bool mfma_fits(const MfmaLaunch& a) {
  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  if (rows_total % G::kTN != 0 || a.kdim % (kStepK * kUnroll) != 0) return false;
  if (a.tile_m < 32 || a.tile_m > G::kTM) return false;
  if (reinterpret_cast<uintptr_t>(a.s) % 16 != 0) return false;
  // Activation rows and output rows are addressed with 32-bit byte offsets.
  const int64_t act_rows = MODE == 0 ? a.n_tok / a.topk : a.n_tok;
  if (act_rows * a.ld_act * 2 > (int64_t)UINT32_MAX - 4096) return false;
  const int64_t out_elt = (MODE == 1 && !a.partial_bf16) ? 4 : 2;
  if ((int64_t)a.n_tok * a.n_out * out_elt > (int64_t)UINT32_MAX - 4096) return false;
  if (a.row_tiles < 1) return false;
  // The DMAs run up to kDW double steps ahead, within the next two row tiles.
  return 2 * (a.kdim / kStepK) > G::kDW;
}

// Work items of one tile (row_tiles row tiles each).
template <int MODE, class G>
__host__ __device__ __forceinline__ int mfma_items_per_tile(const MfmaLaunch& a) {
  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  return (rows_total / G::kTN + a.row_tiles - 1) / a.row_tiles;
}

// Workgroups of an MFMA range sized for `n_tiles` tiles: whole rounds of one
// tile per XCD, mfma_items_per_tile each (mfma_item's block mapping).
template <int MODE, class G>
__host__ __device__ __forceinline__ int64_t mfma_blocks(const MfmaLaunch& a, int n_tiles) {
  return (int64_t)(n_tiles + kXcds - 1) / kXcds * kXcds * mfma_items_per_tile<MODE, G>(a);
}

// The MFMA range of a launch: sized for the most tiles a routing can give.
template <int MODE, class G>
int64_t mfma_grid(const MfmaLaunch& a) {
  return mfma_blocks<MODE, G>(a, a.max_tiles);
}

}  // namespace mfma_dev
}  // namespace
}  // namespace w4a16
