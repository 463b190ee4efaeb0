// Token-to-expert sort with block padding (moe_align_block_size) for gfx950.
//
// Reference: kernels/w4a16_moe.py:187-290 builds the same outputs from ~25
// torch ops (scatter_add_ histogram, cumsum of padded counts, stable sort,
// scatter_reduce amin for the rank, index_put, searchsorted, masked_fill).
// Here it is one workgroup and one launch:
//   1. every wave owns a contiguous chunk of the flat (token, slot) index
//      range and histograms it into its own LDS row cnt[wave][expert];
//   2. a column prefix over the wave rows turns cnt into each wave's
//      starting rank inside every expert (this is what makes the sort stable:
//      earlier chunks rank first);
//   3. a workgroup scan of the padded counts gives the expert offsets;
//   4. every wave walks its chunk again 64 indices at a time; lanes routed to
//      the same expert find each other with ballots over the expert-id bits,
//      take rank = popcount(peers below me) and the lowest peer advances the
//      wave's cursor -- ascending flat index inside an expert, as a stable
//      sort gives;
//   5. padding slots and the tail get the sentinel M*topk, each expert's
//      thread writes the expert id of the blocks it owns (what searchsorted
//      right=True of the block starts over the offsets gives), blocks past
//      the padded end get -1 -- written as soon as the offsets are known,
//      before step 4, so that these stores drain during the placement.
// Integer only; the output is bit-identical to the reference over the whole
// fixed-size buffers.  Ids outside [0, E) are skipped and counted.
#include "common.hpp"

namespace w4a16 {
namespace {

// Workgroup barrier for LDS only: the kernels here share data through LDS
// alone (no thread reads another's global stores), so a barrier waits for
// the wave's LDS accesses and leaves its global loads and stores in flight
// -- a __syncthreads() fence would wait for every one of them (the ids'
// loads while the counts are cleared, the sentinel stores during the
// placement).  The memory clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// NV inclusive scans over the 64 lanes of a wave with DPP lane moves (no
// LDS), step by step over all NV values so that the independent moves fill
// each other's wait states: shifts by 1, 2, 4 and 8 lanes inside each row of
// 16 (lanes without a source add 0), then the last lane of row 0 is added to
// row 1 and of row 2 to row 3 (row_bcast:15), then the last lane of row 1 to
// rows 2 and 3 (row_bcast:31).
template <int NV>
__device__ __forceinline__ void wave_inclusive_scan_n(int (&x)[NV]) {
#define W4A16_SCAN_STEP(CTRL, ROWS, BC)                                        \
  _Pragma("unroll") for (int k = 0; k < NV; ++k)                               \
    x[k] += __builtin_amdgcn_update_dpp(0, x[k], CTRL, ROWS, 0xF, BC);
  W4A16_SCAN_STEP(0x111, 0xF, true)   // row_shr:1
  W4A16_SCAN_STEP(0x112, 0xF, true)   // row_shr:2
  W4A16_SCAN_STEP(0x114, 0xF, true)   // row_shr:4
  W4A16_SCAN_STEP(0x118, 0xF, true)   // row_shr:8
  W4A16_SCAN_STEP(0x142, 0xA, false)  // row_bcast:15
  W4A16_SCAN_STEP(0x143, 0xC, false)  // row_bcast:31
#undef W4A16_SCAN_STEP
}

// NV exclusive scans of one int per thread over the workgroup at once, for
// values that are zero outside waves w0 .. w0 + nv - 1: those waves scan
// their own values, and after one barrier every thread sums the wave totals
// it needs from LDS.  wt is 16-byte aligned LDS of 16 NV ints, not reused
// before the caller's next barrier.  All threads must call.
template <int NV>
__device__ void block_exclusive_scan_n(const int (&v)[NV], int (&excl)[NV], int (&total)[NV],
                                       int* wt, int w0, int nv) {
  static_assert(NV % 4 == 0, "wave totals are read 4 at a time");
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int wr = wid - w0;  // the wave's rank among the scanning waves
  int x[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) x[k] = v[k];
  if (wr >= 0 && wr < nv) {
    wave_inclusive_scan_n<NV>(x);
    if (lane == 63) {
#pragma unroll
      for (int k = 0; k < NV; ++k) wt[wr * NV + k] = x[k];
    }
  }
  lds_barrier();
  int pre[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) pre[k] = total[k] = 0;
  for (int w = 0; w < nv; ++w) {
#pragma unroll
    for (int k4 = 0; k4 < NV; k4 += 4) {
      const int4 t = *reinterpret_cast<const int4*>(wt + w * NV + k4);
      const int tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        total[k4 + k] += tv[k];
        pre[k4 + k] += w < wr ? tv[k] : 0;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) excl[k] = wr < 0 ? 0 : wr < nv ? x[k] - v[k] + pre[k] : total[k];
}

// Token blocks (32 slots) of the tallest MFMA tile: the tile list is ordered
// by height class, tallest first.
constexpr int kTileClasses = kMfmaTileMMax / 32;

// Work lists of the fused call.  An expert with more than gemv_max_tokens
// pairs gets ceil(count / tile_m) MFMA tiles of near-equal size (multiples of
// 32 slots but the last); the tiles are listed by height class, tallest
// first (experts ascending within a class), so that the MFMA launch starts
// its longest tiles first.  Every other routed expert's single sorted block
// goes to the GEMV list.  Thread tid owns experts e0 .. e0 + ipt - 1.
//
// The lists take two parts around one workgroup scan, the one that also
// gives the padded offsets (kScanSlots values per thread):
//   scan_inputs   this thread's tiles per class (slots 0 .. NC - 1), GEMV
//                 blocks (slot NC) and padded pair count (slot NC + 1);
//   write_work_lists  the lists, from the scan's exclusive prefixes and
//                 totals of slots 0 .. NC.
constexpr int kScanSlots = kTileClasses + 2;

// n / d for n >= 0, d >= 1: below 2^22 a float quotient (the hardware
// reciprocal, off from n / d by less than 1) corrected by one step each way
// -- exact, in a few instructions instead of an integer division's ~35.
__device__ __forceinline__ int div_small(int n, int d) {
  if (n >= (1 << 22) || d >= (1 << 22)) return n / d;
  int q = (int)((float)n * __builtin_amdgcn_rcpf((float)d));
  q -= q * d > n ? 1 : 0;
  q += (q + 1) * d <= n ? 1 : 0;
  return q;
}

// Tile height and count of an expert with c > gemv_max_tokens pairs.
__device__ __forceinline__ void tile_split(int c, int tile_m, int& per, int& n_t) {
  const int n_ch = div_small(c + tile_m - 1, tile_m);
  per = (div_small(c + n_ch - 1, n_ch) + 31) & ~31;  // <= tile_m
  n_t = div_small(c + per - 1, per);
}

// c rounded up to a multiple of the block size B.
__device__ __forceinline__ int round_up_block(int c, int B) {
  return div_small(c + B - 1, B) * B;
}

__device__ void scan_inputs(const AlignLaunch& a, const int32_t* tot, int e0, int ipt,
                            int (&v)[kScanSlots]) {
  constexpr int NC = kTileClasses;
  const int E = a.num_experts, B = a.block, thr = a.gemv_max_tokens;
  // class of a tile of n slots: NC - (token blocks)
  auto cls = [](int n) { return NC - ((n + 31) >> 5); };
#pragma unroll
  for (int k = 0; k < kScanSlots; ++k) v[k] = 0;
  for (int i = 0; i < ipt; ++i) {
    const int e = e0 + i;
    if (e >= E) break;
    const int c = tot[e];
    v[NC + 1] += round_up_block(c, B);
    if (!a.tiles) continue;
    if (c > thr) {
      int per, n_t;
      tile_split(c, a.tile_m, per, n_t);
      const int kf = cls(per), kl = cls(c - (n_t - 1) * per);
#pragma unroll
      for (int k = 0; k < NC; ++k) v[k] += (k == kf ? n_t - 1 : 0) + (k == kl ? 1 : 0);
    } else if (c > 0) {
      ++v[NC];
    }
  }
}

__device__ void write_work_lists(const AlignLaunch& a, const int32_t* tot, const int32_t* off,
                                 int e0, int ipt, const int (&excl)[kScanSlots],
                                 const int (&total)[kScanSlots], bool scalars) {
  constexpr int NC = kTileClasses;
  const int E = a.num_experts, B = a.block, thr = a.gemv_max_tokens;
  auto cls = [](int n) { return NC - ((n + 31) >> 5); };
  int pos[NC + 1];
  int n_tiles = 0;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    pos[k] = excl[k] + n_tiles;
    n_tiles += total[k];
  }
  pos[NC] = excl[NC];
  for (int i = 0; i < ipt; ++i) {
    const int e = e0 + i;
    if (e >= E) break;
    const int c = tot[e];
    if (c > thr) {
      int per, n_t;
      tile_split(c, a.tile_m, per, n_t);
      for (int s0 = 0; s0 < c; s0 += per) {
        const int n = min(per, c - s0);
        const int k = cls(n);
        int p = 0;
#pragma unroll
        for (int j = 0; j < NC; ++j)
          if (j == k) p = pos[j]++;
        a.tiles[p] = make_int4(e, off[e] + s0, n, 0);
      }
    } else if (c > 0) {
      a.gemv_blocks[pos[NC]++] = div_small(off[e], B);
    }
  }
  if (scalars) {
    a.n_tiles[0] = n_tiles;
    a.n_gemv[0] = total[NC];
  }
}

// The padding of the sorted ids and of the block experts, by threads t of nt
// (the whole workgroup), once the counts and offsets are known:
//   * expert e's padding slots off[e] + tot[e] .. off[e+1] - 1 get the
//     sentinel from tpe = max(1, nt / E) threads, every tpe-th slot each;
//   * the tail slots from the padded total on get it too, 16 bytes per store
//     where the buffer is 16-byte aligned;
//   * blocks from the padded total on get expert -1.
__device__ void write_padding(const AlignLaunch& a, const int32_t* tot, const int32_t* off,
                              int total, int t, int nt) {
  const int E = a.num_experts, B = a.block, sent = a.n_tok, em = a.em;
  int32_t* const sorted = a.sorted;
  const int tpe = max(1, div_small(nt, E));
  for (int idx = t; idx < E * tpe; idx += nt) {
    const int e = div_small(idx, tpe);
    for (int p = off[e] + tot[e] + (idx - e * tpe); p < off[e + 1]; p += tpe) sorted[p] = sent;
  }
  int p4 = em;  // start of the 16-byte stores (none when unaligned)
  if ((reinterpret_cast<uintptr_t>(sorted) & 15) == 0) {
    p4 = min(em, (total + 3) & ~3);
    const int n4 = (em - p4) >> 2;
    const int4 s4 = make_int4(sent, sent, sent, sent);
    for (int i = t; i < n4; i += nt) reinterpret_cast<int4*>(sorted + p4)[i] = s4;
    for (int p = p4 + 4 * n4 + t; p < em; p += nt) sorted[p] = sent;
  }
  for (int p = total + t; p < p4; p += nt) sorted[p] = sent;
  for (int b = div_small(total, B) + t; b < a.n_blocks; b += nt) a.expert_ids[b] = -1;
}

// Block b's expert for the blocks of experts e0 .. e0 + ipt - 1: expert e
// owns blocks off[e] / B .. off[e+1] / B - 1 (the offsets are multiples of
// B), so each expert's thread writes its own -- the searchsorted(right) of
// the reference's block starts over the offsets, without a search per block.
__device__ void write_block_experts(const AlignLaunch& a, const int32_t* off, int e0, int ipt) {
  const int B = a.block, E = a.num_experts;
  for (int i = 0; i < ipt; ++i) {
    const int e = e0 + i;
    if (e >= E) break;
    const int b1 = min(div_small(off[e + 1], B), a.n_blocks);
    for (int b = div_small(off[e], B); b < b1; ++b) a.expert_ids[b] = e;
  }
}

__global__ __launch_bounds__(1024) void align_kernel(const AlignLaunch a) {
  extern __shared__ int32_t smem[];
  __shared__ __align__(16) int32_t scan_tot[kScanSlots * 16];
  __shared__ int32_t s_drop;

  const int nthr = blockDim.x;
  const int nw = nthr >> 6;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int E = a.num_experts;
  const int B = a.block;
  const int n_tok = a.n_tok;

  int32_t* cnt = smem;           // [nw][E]
  int32_t* off = cnt + nw * E;   // [E+1]
  int32_t* tot = off + E + 1;    // [E]

  // Contiguous chunk of flat indices per wave, a multiple of 64.
  const int per = ((n_tok + nw - 1) / nw + 63) & ~63;
  const int beg = min(n_tok, wid * per);
  const int end = min(n_tok, beg + per);

  // Ids are read kBatch * 64 at a time per wave, every load issued before
  // the first is used: one memory latency per batch, not per 64 ids.
  constexpr int kBatch = 8;
  // Lanes past the wave's end load a clamped (in-bounds) entry; both walks
  // below test f < end before using a value, so nothing here waits for the
  // loads.
  auto load_batch = [&](int f0, int (&ev)[kBatch]) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int f = f0 + 64 * u + lane;
      ev[u] = a.ids[min(f, max(end - 1, 0))];
    }
  };

  // A wave's share of at most one batch (every call below the many-workgroup
  // sort's size) is loaded once and kept in registers for the placement.  A
  // wave with no ids loads nothing (with no pairs at all the id buffer is
  // empty, and load_batch's clamped index would still read entry 0); its
  // loops below do not run.
  const bool one_batch = end - beg <= 64 * kBatch;  // uniform
  int ev1[kBatch];
  if (one_batch && beg < end) load_batch(beg, ev1);

  // (the ids' loads are in flight while the counts are cleared)
  for (int i = tid; i < nw * E; i += nthr) cnt[i] = 0;
  if (tid == 0) s_drop = 0;
  lds_barrier();

  // 1. per-wave histogram
  int drop = 0;
  for (int f0 = beg; f0 < end; f0 += 64 * kBatch) {
    int ev[kBatch];
    if (one_batch) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) ev[u] = ev1[u];
    } else {
      load_batch(f0, ev);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (f0 + 64 * u >= end) break;  // uniform
      const int f = f0 + 64 * u + lane;
      const int e = ev[u];
      if (f < end) {
        if (e >= 0 && e < E)
          atomicAdd(&cnt[wid * E + e], 1);
        else
          ++drop;
      }
    }
  }
  if (drop) atomicAdd(&s_drop, drop);
  lds_barrier();

  // 2. column prefix over waves: cnt[w][e] <- rank of wave w's first pair
  for (int e = tid; e < E; e += nthr) {
    int run = 0;
    for (int w = 0; w < nw; ++w) {
      const int c = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += c;
    }
    tot[e] = run;
  }
  lds_barrier();

  // 3. offsets = exclusive scan of counts rounded up to the block size, in
  // the same workgroup scan as the work lists' counts.  The experts belong to
  // n_own threads (ipt each, ascending): the workgroup's last ones when their
  // waves hold no ids, so that the expert-parallel writes after the scan
  // overlap the placement, else its first ones.
  const int ipt = (E + nthr - 1) / nthr;
  const int n_own = (E + ipt - 1) / ipt;
  const int own_waves = (n_own + 63) >> 6;
  const bool own_last = (n_tok + per - 1) / per <= nw - own_waves;
  const int own0 = own_last ? nthr - n_own : 0;  // first owner thread
  const int own = tid - own0;                    // in [0, n_own): an owner
  const int e0 = own >= 0 && own < n_own ? own * ipt : E;
  int sv[kScanSlots], sx[kScanSlots], st[kScanSlots];
  scan_inputs(a, tot, e0, ipt, sv);
  block_exclusive_scan_n<kScanSlots>(sv, sx, st, scan_tot, own0 >> 6,
                                     own_last ? nw - (own0 >> 6) : own_waves);
  const int total = st[kScanSlots - 1];
  int excl = sx[kScanSlots - 1];
  for (int i = 0; i < ipt; ++i) {
    const int e = e0 + i;
    if (e < E) {
      off[e] = excl;
      excl += round_up_block(tot[e], B);
    }
  }
  if (own == 0) off[E] = total;
  lds_barrier();

  // 3b. the outputs that need only the counts and offsets: the owners' work
  // lists of the fused call, block experts and scalars, everyone's share of
  // the padding -- while the placement writes the other sorted positions
  if (own >= 0 && own < n_own) {
    if (a.tiles) write_work_lists(a, tot, off, e0, ipt, sx, st, own == 0);
    write_block_experts(a, off, e0, ipt);
    if (a.offsets)
      for (int e = own; e <= E; e += n_own) a.offsets[e] = off[e];
    if (own == 0) {
      a.num_post[0] = total;
      if (a.dropped) a.dropped[0] = s_drop;
    }
  }
  write_padding(a, tot, off, total, tid, nthr);

  // 4. stable placement: the pair's slot is its expert's offset plus its rank
  // (cnt holds each wave's next rank inside every expert)
  int ebits = 0;
  while ((1 << ebits) < E) ++ebits;
  const uint64_t lt = lanemask_lt();
  for (int fb = beg; fb < end; fb += 64 * kBatch) {
    int ev[kBatch];
    if (one_batch) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) ev[u] = ev1[u];
    } else {
      load_batch(fb, ev);
    }
    // the 64-id groups in ascending order: each advances the wave's cursors
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (fb + 64 * u >= end) break;  // uniform
      const int f = fb + 64 * u + lane;
      const int e = ev[u];
      const bool ok = f < end && e >= 0 && e < E;
      uint64_t peers = ballot(ok);
      for (int bit = 0; bit < ebits; ++bit) {
        const bool set = ok && ((e >> bit) & 1);
        const uint64_t m = ballot(set);
        peers &= set ? m : ~m;
      }
      int base = 0, eoff = 0;
      if (ok) base = cnt[wid * E + e], eoff = off[e];
      __builtin_amdgcn_wave_barrier();
      if (ok) {
        const uint64_t below = peers & lt;
        a.sorted[eoff + base + __popcll(below)] = f;
        if (below == 0) cnt[wid * E + e] = base + __popcll(peers);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }

}

// ---- many workgroups (large batches) --------------------------------------
// The flat index range is cut into chunks of kChunk pairs, one workgroup of
// kChunk / 64 waves each, so every wave places a single batch of 64 pairs:
//   align_count_kernel  per chunk, the pairs of each expert -> ctot[chunk][E]
//                       and the chunk's dropped pairs -> cdrop[chunk];
//   align_place_kernel  per chunk, the expert totals and the chunk's starting
//                       rank in every expert (sums over the earlier chunks),
//                       the padded offsets, and the stable placement of the
//                       chunk's pairs; workgroup 0 also writes the padding
//                       sentinels, the block experts, the work lists and the
//                       scalars.
// The result is the same function as align_kernel's.
constexpr int kChunk = 1024;
constexpr int kChunkWaves = kChunk / 64;
static_assert(kAlignChunkedMaxE <= kChunk, "one part of the threads covers every expert");

__global__ __launch_bounds__(kChunk) void align_count_kernel(const AlignLaunch a,
                                                             int32_t* ctot, int32_t* cdrop) {
  extern __shared__ int32_t hist[];  // [E]
  const int E = a.num_experts;
  const int tid = threadIdx.x;
  for (int i = tid; i <= E; i += kChunk) hist[i] = 0;
  lds_barrier();
  const int f = blockIdx.x * kChunk + tid;
  int drop = 0;
  if (f < a.n_tok) {
    const int e = a.ids[f];
    if (e >= 0 && e < E)
      atomicAdd(&hist[e], 1);
    else
      drop = 1;
  }
  // dropped pairs of the chunk: one wave-level ballot count per wave
  const int wd = __popcll(ballot(drop != 0));
  lds_barrier();
  if ((tid & 63) == 0 && wd) atomicAdd(&hist[E], wd);
  lds_barrier();
  for (int i = tid; i < E; i += kChunk) ctot[(int64_t)blockIdx.x * E + i] = hist[i];
  if (tid == 0) cdrop[blockIdx.x] = hist[E];
}

__global__ __launch_bounds__(kChunk) void align_place_kernel(const AlignLaunch a,
                                                             const int32_t* ctot,
                                                             const int32_t* cdrop) {
  extern __shared__ int32_t smem[];
  __shared__ __align__(16) int32_t scan_tot[kScanSlots * 16];
  constexpr int nw = kChunkWaves;
  const int tid = threadIdx.x;
  const int wid = tid >> 6;
  const int E = a.num_experts;
  const int B = a.block;
  const int n_tok = a.n_tok;
  const int n_chunks = gridDim.x;
  const int g = blockIdx.x;

  int32_t* cnt = smem;           // [nw][E]
  int32_t* off = cnt + nw * E;   // [E+1]
  int32_t* tot = off + E + 1;    // [E]

  // 1. expert totals and this chunk's starting rank in every expert: the
  // threads split into parts of E, part p summing chunks p, p + parts, ...
  // (independent loads in flight), combined with LDS atomics
  for (int i = tid; i < nw * E; i += kChunk) cnt[i] = 0;
  for (int e = tid; e < E; e += kChunk) tot[e] = off[e] = 0;
  lds_barrier();
  {
    const int parts = max(1, kChunk / E);
    const int part = tid / E;
    const int e = tid - part * E;
    if (part < parts) {
      int before = 0, all = 0;
      // 16 chunks' counts in flight per round trip (a batch of 40 chunks,
      // M=4096, is one round trip on four parts)
      constexpr int kLoads = 16;
      for (int c0 = part; c0 < n_chunks; c0 += kLoads * parts) {
        int v[kLoads];
#pragma unroll
        for (int b = 0; b < kLoads; ++b) {
          const int c = c0 + b * parts;
          v[b] = c < n_chunks ? ctot[(int64_t)c * E + e] : 0;
        }
#pragma unroll
        for (int b = 0; b < kLoads; ++b) {
          before += c0 + b * parts < g ? v[b] : 0;
          all += v[b];
        }
      }
      atomicAdd(&tot[e], all);
      atomicAdd(&off[e], before);  // parked here until the offsets are known
    }
  }
  lds_barrier();

  // 2. this chunk's per-wave histograms (wave w: pairs 64 w .. of the chunk)
  const int f = g * kChunk + tid;
  const int e_me = f < n_tok ? a.ids[f] : -1;
  const bool ok = f < n_tok && e_me >= 0 && e_me < E;
  if (ok) atomicAdd(&cnt[wid * E + e_me], 1);
  lds_barrier();

  // 3. column prefix over the waves, on top of the chunk's starting rank
  for (int e = tid; e < E; e += kChunk) {
    int run = off[e];
    for (int w = 0; w < nw; ++w) {
      const int c = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += c;
    }
  }
  lds_barrier();

  // 4. offsets = exclusive scan of the padded totals, in the same workgroup
  // scan as the work lists' counts (which workgroup 0 writes)
  const int ipt = (E + kChunk - 1) / kChunk;
  const int e0 = tid * ipt;
  int sv[kScanSlots], sx[kScanSlots], st[kScanSlots];
  scan_inputs(a, tot, e0, ipt, sv);
  // the owners (e0 < E) are threads 0 .. ceil(E / ipt) - 1
  block_exclusive_scan_n<kScanSlots>(sv, sx, st, scan_tot, 0, ((E + ipt - 1) / ipt + 63) >> 6);
  const int total = st[kScanSlots - 1];
  int excl = sx[kScanSlots - 1];
  for (int i = 0; i < ipt; ++i) {
    const int e = e0 + i;
    if (e < E) {
      off[e] = excl;
      excl += round_up_block(tot[e], B);
    }
  }
  if (tid == 0) off[E] = total;
  lds_barrier();

  // 5. stable placement: lanes routed to the same expert find each other
  // with ballots over the expert-id bits and take their rank among them
  int ebits = 0;
  while ((1 << ebits) < E) ++ebits;
  uint64_t peers = ballot(ok);
  for (int bit = 0; bit < ebits; ++bit) {
    const bool set = ok && ((e_me >> bit) & 1);
    const uint64_t m = ballot(set);
    peers &= set ? m : ~m;
  }
  if (ok) a.sorted[off[e_me] + cnt[wid * E + e_me] + __popcll(peers & lanemask_lt())] = f;
  if (g != 0) return;

  // 6. workgroup 0: work lists, sentinels, block experts, scalars
  if (a.tiles) write_work_lists(a, tot, off, e0, ipt, sx, st, tid == 0);
  write_block_experts(a, off, e0, ipt);
  write_padding(a, tot, off, total, tid, kChunk);
  if (a.offsets)
    for (int e = tid; e <= E; e += kChunk) a.offsets[e] = off[e];
  if (tid == 0) {
    a.num_post[0] = total;
    if (a.dropped) {
      int d = 0;
      for (int c = 0; c < n_chunks; ++c) d += cdrop[c];
      a.dropped[0] = d;
    }
  }
}

}  // namespace

int align_chunks(int n_tok) { return (n_tok + kChunk - 1) / kChunk; }

hipError_t launch_align(const AlignLaunch& a, hipStream_t stream) {
  if (a.chunk_scratch && a.n_tok >= kAlignChunkedMinPairs && a.num_experts <= kAlignChunkedMaxE) {
    const int n_chunks = align_chunks(a.n_tok);
    int32_t* ctot = a.chunk_scratch;
    int32_t* cdrop = a.chunk_scratch + (size_t)n_chunks * a.num_experts;
    hipLaunchKernelGGL(align_count_kernel, dim3(n_chunks), dim3(kChunk),
                       sizeof(int32_t) * ((size_t)a.num_experts + 1), stream, a, ctot, cdrop);
    const size_t lds = sizeof(int32_t) * ((size_t)kChunkWaves * a.num_experts +
                                          2 * (size_t)a.num_experts + 1);
    hipLaunchKernelGGL(align_place_kernel, dim3(n_chunks), dim3(kChunk), lds, stream, a, ctot,
                       cdrop);
    return hipGetLastError();
  }
  const int threads = a.num_experts <= 512 ? 1024 : 512;
  const int nw = threads / 64;
  const size_t lds =
      sizeof(int32_t) * ((size_t)nw * a.num_experts + 2 * (size_t)a.num_experts + 1);
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(threads), lds, stream, a);
  return hipGetLastError();
}

}  // namespace w4a16
