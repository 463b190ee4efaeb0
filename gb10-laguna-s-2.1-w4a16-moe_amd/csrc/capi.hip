// C ABI of the W4A16 MoE library: argument checks, workspace layout and the
// launch sequence align -> w13 -> w2 -> combine, all on the caller's stream
// (no align for small batches, whose GEMV kernels route themselves).
#include <limits.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "../../include/w4a16_moe.h"
#include "common.hpp"

using namespace w4a16;

namespace {

constexpr size_t kWsAlign = 256;
constexpr int64_t kMaxExperts = 1024;
constexpr int64_t kMaxTopk = 256;

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int align_sizes(int64_t M, int64_t topk, int64_t E, int64_t block, int64_t* em,
                int64_t* nb) {
  if (block < 1) return W4A16_ERR_INVALID_BLOCK;
  if (M < 0 || topk < 1 || E < 1) return W4A16_ERR_INVALID_SHAPE;
  if (topk > kMaxTopk || E > kMaxExperts) return W4A16_ERR_INVALID_SHAPE;
  if (block > (int64_t)INT_MAX / (kMaxExperts + 1)) return W4A16_ERR_INVALID_BLOCK;
  const int64_t n_tok = M * topk;
  const int64_t padded = n_tok + E * (block - 1);
  const int64_t e_m = (padded + block - 1) / block * block;
  if (n_tok > INT_MAX / 2 || e_m > INT_MAX / 2) return W4A16_ERR_INVALID_SHAPE;
  *em = e_m;
  *nb = e_m / block;
  return W4A16_OK;
}

// Dispatch choices of one call: the public w4a16_moe_tuning, resolved.
struct Tuning {
  int gemv_only_max_m;  // M at or below this: every expert on the GEMV kernels
  int gemv_max_tokens;  // above it: experts with more pairs go to MFMA tiles
  int tc;               // GEMV token rows per pass (0 = launcher's choice)
  int tile_m;           // MFMA tile height (0 = built-in, see compute_layout)
  int upw;              // GEMV row slabs per workgroup (0 = launcher's choice)
  int lpr;              // GEMV lanes per weight row (0 = launcher's choice)
  int w2_fused_max_m;   // M at or below this: w2 and the top-k sum as one kernel
  bool auto_split;      // gemv_max_tokens is the built-in choice (see compute_layout)
  int row_tiles;        // 256-row weight blocks per MFMA work item (0 = built-in per GEMM)
};

struct Layout {
  size_t off[W4A16_WS_NFIELDS];
  size_t total;
  int64_t em, nb;
  bool mfma;          // heavy experts run on the MFMA kernels
  bool gemv;          // the GEMV kernels run (they may find no work)
  bool chunked;       // the sort runs over many workgroups (chunk counts at off_chunks)
  size_t off_chunks;
  bool route;         // GEMV kernels route themselves; no align kernel
  int tile_m;         // MFMA tile height (slots)
  int64_t max_tiles;  // bound of the MFMA tile list
  int64_t max_gemv;   // bound of the GEMV block list / GEMV work items
  int64_t max_items;  // self-routed work items: one per (token, slot) pair
  bool token;         // one token: w2 and the combine in one launch
  bool partial_bf16;  // PARTIAL holds bf16 rows (else fp32)
  int gemv_max_tokens;
  int tc;
  int upw;
  int lpr;
  int row_tiles_w13;  // 256-row weight blocks per MFMA work item
  int row_tiles_w2;
};

// An expert with more than this many (token, slot) pairs runs on MFMA tiles;
// the others stay on the GEMV kernels.  Must stay below the sort block (16).
constexpr int kGemvMaxTokens = W4A16_GEMV_MAX_TOKENS;
constexpr int kGemvOnlyMaxM = W4A16_GEMV_ONLY_MAX_M;
// Self-routed calls up to this many tokens run w2 and the top-k sum as one
// kernel.  Measured on MI355X (E=256, top-10): M=2 28.6 vs 30.9 us, M=4
// 48.1 vs 49.1 us (skewed routing 40.9 vs 44.7); at M=8 the experts shared
// by tokens, read once per token, cancel the saved launch.
constexpr int kW2FusedMaxM = 4;
// The reference keeps the top-k-weighted w2 rows in a bf16 buffer
// (kernels/w4a16_moe.py:311) and sums them in fp32, except for calls of at
// most this many tokens, which accumulate them in fp32 (:763).  The partial
// rows here follow the same rounding points.
constexpr int64_t kFp32PartialMaxM = 4;
// The split dispatch runs each GEMM's GEMV and MFMA work items as one mixed
// launch where a mixed kernel covers the shapes (0: always two launches;
// overridable at build time for measurements).
#ifndef W4A16_MIXED_LAUNCHES
#define W4A16_MIXED_LAUNCHES 1
#endif
constexpr bool kMixedLaunches = W4A16_MIXED_LAUNCHES != 0;
// Row tiles (256 weight rows) one MFMA workgroup runs in turn for one token
// tile (a work item): the loads stream on across them, so the latency of a
// workgroup's first loads is paid once per item, at the price of fewer and
// longer items.  Built-in choice: the divisor of the row-tile count nearest
// (in ratio) item_work / (double steps x token blocks per tile), so that an
// item holds about item_work MFMA block-steps per wave (w13 330, w2 180: w2
// rows write twice the outputs), with at least two items per CU left for
// balance.  Measured on MI355X (E=256, top-10,
// K=3072, N=1024), best per GEMM: M=4096 w13 1 (578 us vs 597 at 2), w2 2
// (371 vs 394 at 1); M=1024 w13 4 (283 vs 331 at 1), w2 6 (161 vs 211 at
// 1); skewed M=64 w13 1 (99 vs 118 at 4).  Every choice is bit-identical.
// These are the 192- and 128-slot tiles; the 64-slot tiles use
// kSmallItemRows* below.
constexpr double kItemWorkW13 = 330.0;
constexpr double kItemWorkW2 = 180.0;
constexpr int64_t kCUs = 256;  // MI355X
// Built-in weight rows per work item of the 64-slot tiles (4-wave
// workgroups, 128-row row tiles).  Measured on MI355X (E=256, top-10,
// K=3072, N=1024) over M=32-512, uniform and skewed routing, 128, 256 or 512
// rows per item: w2 is fastest at 512 everywhere (5-10 % below 128: skewed
// M=64 40.7 vs 44.8 us, uniform M=192 113 vs 123 us), w13 at 256 or within
// 1 % of it (uniform M=256 228 vs 237 us against 128).
constexpr int64_t kSmallItemRowsW13 = 256;
constexpr int64_t kSmallItemRowsW2 = 512;

int pick_row_tiles(int64_t n_tiles_n, int64_t steps, int64_t n_tok, int64_t E,
                   double item_work) {
  const double avg = (double)n_tok / (double)E;
  const double blocks = std::min(6.0, std::max(1.0, std::ceil(avg / 32.0)));
  const double want = item_work / ((double)steps * blocks);
  // items: an estimate of the MFMA tiles (an expert's tile needs > 4 pairs)
  const int64_t est_tiles = std::max<int64_t>(1, std::min<int64_t>(E, n_tok / 8));
  int best = 1;
  double best_d = 1e30;
  for (int r = 1; r <= n_tiles_n && r <= 16; ++r) {
    if (n_tiles_n % r) continue;
    if (r > 1 && est_tiles * (n_tiles_n / r) < 2 * kCUs) break;
    const double d = std::fabs(std::log((double)r / want));
    if (d < best_d) best_d = d, best = r;
  }
  return best;
}
// The largest divisor of n_blocks (256-row weight blocks of a GEMM) of at
// most `rows` weight rows.
int small_row_tiles(int64_t n_blocks, int64_t rows) {
  int best = 1;
  for (int r = 1; r <= n_blocks && r * (int64_t)kMfmaTileN <= rows; ++r)
    if (n_blocks % r == 0) best = r;
  return best;
}
// Average (token, slot) pairs per expert from which the built-in split sends
// every expert to the MFMA kernels (gemv_max_tokens 0, no GEMV launches).
constexpr int64_t kAllMfmaMinPairs = 32;
// Average pairs per expert below which the built-in MFMA tile is 128 slots.
// Measured on MI355X (E=256, top-10): M=256 skewed 307 vs 406 us, M=1024
// 505 vs 552 us; at M=4096 192 wins (1049 vs 1171 us uniform).
constexpr int64_t kTile128MaxPairs = 64;
// Average pairs per expert below which the built-in MFMA tile is 64 slots:
// under skewed routing a hot expert then becomes more, shorter tiles.
// Measured on MI355X (E=256, top-10): M=256 skewed 258 vs 323 us (tile 128)
// and 411 us (192); uniform routing from M=64 to 512 within 1 % of the
// other heights; M=1024 uniform 474 vs 464 us (128).
constexpr int64_t kTile64MaxPairs = 24;

int check_gemm_shape(int64_t N, int64_t K, int64_t group) {
  if (N <= 0 || K <= 0) return W4A16_ERR_INVALID_SHAPE;
  if (group != 32 && group != 64 && group != 128) return W4A16_ERR_UNSUPPORTED_GROUP;
  if (K % group != 0 || N % group != 0) return W4A16_ERR_UNSUPPORTED_GROUP;
  if (K % 32 != 0 || N % 32 != 0) return W4A16_ERR_INVALID_SHAPE;
  // one staged activation row (K or N bf16 values) must fit in LDS
  if (K > 16384 || N > 16384) return W4A16_ERR_INVALID_SHAPE;
  return W4A16_OK;
}

Tuning default_tuning() {
  return Tuning{kGemvOnlyMaxM, kGemvMaxTokens, 0, 0, 0, 0, kW2FusedMaxM, true, 0};
}

// NULL selects the built-in choices.
int resolve_tuning(const w4a16_moe_tuning* t, Tuning* out) {
  *out = default_tuning();
  if (!t) return W4A16_OK;
  if (t->mfma_row_tiles < 0 || t->mfma_row_tiles > 16) return W4A16_ERR_INVALID_TUNING;
  out->row_tiles = t->mfma_row_tiles;
  if (t->w2_fused_max_m < 0) return W4A16_ERR_INVALID_TUNING;
  if (t->w2_fused_max_m > 0) out->w2_fused_max_m = t->w2_fused_max_m;
  const int lpr = t->gemv_lanes_per_row;
  if (lpr != 0 && lpr != 8 && lpr != 32) return W4A16_ERR_INVALID_TUNING;
  out->lpr = lpr;
  if (t->gemv_only_max_m < 0) return W4A16_ERR_INVALID_TUNING;
  if (t->gemv_max_tokens < 0 || t->gemv_max_tokens >= W4A16_FUSED_BLOCK_M)
    return W4A16_ERR_INVALID_TUNING;
  const int tc = t->gemv_tokens_per_pass;
  if (tc != 0 && tc != 1 && tc != 2 && tc != 4) return W4A16_ERR_INVALID_TUNING;
  const int tm = t->mfma_tile_m;
  if (tm != 0 && tm != kMfmaTileMSmall && tm != kMfmaTileMMin && tm != kMfmaTileMMax)
    return W4A16_ERR_INVALID_TUNING;
  if (tm != 0) out->tile_m = tm;
  const int upw = t->gemv_units_per_wg;
  if (upw != 0 && upw != 1 && upw != 2 && upw != 4) return W4A16_ERR_INVALID_TUNING;
  out->upw = upw;
  out->gemv_only_max_m = t->gemv_only_max_m;
  out->gemv_max_tokens = t->gemv_max_tokens;
  out->auto_split = false;
  out->tc = tc;
  return W4A16_OK;
}

// mfma_ok = false keeps every expert on the GEMV kernels (the MFMA kernels
// read the scales in 16-byte pieces and need them 16-byte aligned).
int compute_layout(int64_t M, int64_t topk, int64_t E, int64_t N, int64_t K,
                   int64_t group, const Tuning& T, Layout* L, bool mfma_ok = true) {
  int st = check_gemm_shape(N, K, group);
  if (st) return st;
  st = align_sizes(M, topk, E, W4A16_FUSED_BLOCK_M, &L->em, &L->nb);
  if (st) return st;
  const size_t n_tok = (size_t)(M * topk);
  // MFMA tiles need whole 256-row weight tiles and whole 256-element weight
  // slabs on both GEMMs; small batches cannot give an expert enough pairs to
  // pay for the extra launches.
  L->mfma = mfma_ok && M > T.gemv_only_max_m && N % kMfmaTileN == 0 && K % kMfmaTileN == 0;
  L->gemv_max_tokens = T.gemv_max_tokens;
  // Built-in split: once experts average 32 or more pairs, an expert with at
  // most gemv_max_tokens of them is vanishingly rare, and the two GEMV
  // launches that would look for one cost more than an MFMA tile for it, so
  // every expert goes to the MFMA kernels and the GEMV launches are skipped.
  if (L->mfma && T.auto_split && (int64_t)n_tok >= kAllMfmaMinPairs * E) L->gemv_max_tokens = 0;
  L->gemv = !L->mfma || L->gemv_max_tokens > 0;
  L->tc = T.tc;
  L->upw = T.upw;
  L->lpr = T.lpr;
  const int64_t heavy = std::min<int64_t>(E, (int64_t)n_tok / (T.gemv_max_tokens + 1));
  // Built-in tile height: 128 slots while experts average fewer than 64
  // pairs (more, shorter tiles: an expert's long tile is the tail of the
  // launch under skewed routing), 192 from there.
  L->tile_m = T.tile_m ? T.tile_m
                       : ((int64_t)n_tok < kTile64MaxPairs * E    ? kMfmaTileMSmall
                          : (int64_t)n_tok < kTile128MaxPairs * E ? kMfmaTileMMin
                                                                  : kMfmaTileMMax);
  if (T.row_tiles > 0) {
    L->row_tiles_w13 = L->row_tiles_w2 = T.row_tiles;
  } else if (L->tile_m <= kMfmaTileMSmall) {
    L->row_tiles_w13 = small_row_tiles(2 * N / kMfmaTileN, kSmallItemRowsW13);
    L->row_tiles_w2 = small_row_tiles(K / kMfmaTileN, kSmallItemRowsW2);
  } else {
    L->row_tiles_w13 = pick_row_tiles(2 * N / kMfmaTileN, K / 64, n_tok, E, kItemWorkW13);
    L->row_tiles_w2 = pick_row_tiles(K / kMfmaTileN, N / 64, n_tok, E, kItemWorkW2);
  }
  L->max_tiles = L->mfma ? (int64_t)n_tok / L->tile_m + heavy : 0;
  L->max_gemv = L->mfma ? std::min<int64_t>(std::min<int64_t>(E, (int64_t)n_tok), L->nb)
                        : std::min<int64_t>((int64_t)n_tok, L->nb);
  // Small batches: the GEMV kernels route themselves from topk_ids (work
  // item = one routed expert), so the align kernel is not run.
  L->route = !L->mfma && M >= 1 && M <= T.gemv_only_max_m &&
             gemv_route_fits((int)n_tok, (int)E, (int)K, (int)N);
  L->max_items = L->route ? (int64_t)n_tok : 0;
  L->token = L->route && M <= T.w2_fused_max_m && w2_token_fits((int)topk, (int)K, (int)N);
  L->partial_bf16 = M > kFp32PartialMaxM;
  size_t cur = 0;
  auto put = [&](int field, size_t bytes) {
    L->off[field] = cur;
    cur = round_up(cur + bytes, kWsAlign);
  };
  put(W4A16_WS_HEADER, 64 * sizeof(int32_t));
  put(W4A16_WS_SORTED_IDS, (size_t)L->em * sizeof(int32_t));
  put(W4A16_WS_EXPERT_IDS, (size_t)L->nb * sizeof(int32_t));
  put(W4A16_WS_OFFSETS, (size_t)(E + 1) * sizeof(int32_t));
  put(W4A16_WS_INTER, n_tok * (size_t)N * sizeof(uint16_t));
  put(W4A16_WS_PARTIAL, n_tok * (size_t)K * (L->partial_bf16 ? sizeof(uint16_t) : sizeof(float)));
  put(W4A16_WS_TILES, (size_t)std::max<int64_t>(L->max_tiles, 1) * 4 * sizeof(int32_t));
  put(W4A16_WS_GEMV_BLOCKS, (size_t)std::max<int64_t>(L->max_gemv, 1) * sizeof(int32_t));
  // Internal (not one of the public fields): the chunk counts of the
  // many-workgroup sort of large batches.
  L->chunked = !L->route && (int64_t)n_tok >= kAlignChunkedMinPairs && E <= kAlignChunkedMaxE;
  L->off_chunks = cur;
  if (L->chunked) cur = round_up(cur + align_chunk_scratch_ints((int)n_tok, (int)E) * 4, kWsAlign);
  L->total = cur;
  return W4A16_OK;
}

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

struct FusedArgs {
  const void* hidden;
  int64_t ld_hidden;
  const void* w13;
  const void* w2;
  const void* s13;
  const void* s2;
  const float* topk_w;
  const int32_t* ids;
  int64_t M, topk, E, N, K, group;
  void* out;
  int64_t ld_out;
  void* ws;
  size_t ws_bytes;
  const w4a16_moe_tuning* tuning;  // null: built-in choices
};

// The MFMA kernels address activation and output rows with 32-bit byte
// offsets from the buffer base: the hidden rows (w13 input), the
// intermediate rows (w13 output, w2 input) and the partial rows (w2 output)
// must each lie below this.
constexpr int64_t kMfmaActBytesMax = (int64_t)UINT32_MAX - 4096;

bool mfma_act_fits(int64_t M, int64_t topk, int64_t N, int64_t K, int64_t ld_hidden) {
  const int64_t partial_elt = M > kFp32PartialMaxM ? 2 : 4;
  return M * ld_hidden * 2 <= kMfmaActBytesMax && M * topk * N * 2 <= kMfmaActBytesMax &&
         M * topk * K * partial_elt <= kMfmaActBytesMax;
}

int validate(const FusedArgs& a, Layout* L) {
  Tuning T;
  int st = resolve_tuning(a.tuning, &T);
  if (st) return st;
  const bool scales16 = aligned(a.s13, 16) && aligned(a.s2, 16);
  st = compute_layout(a.M, a.topk, a.E, a.N, a.K, a.group, T, L, scales16);
  if (st) return st;
  if (a.M == 0) return W4A16_OK;
  if (!a.hidden || !a.w13 || !a.w2 || !a.s13 || !a.s2 || !a.topk_w || !a.ids ||
      !a.out || !a.ws)
    return W4A16_ERR_NULL_POINTER;
  if (a.ld_hidden < a.K || a.ld_out < a.K) return W4A16_ERR_INVALID_SHAPE;
  if (L->mfma && !mfma_act_fits(a.M, a.topk, a.N, a.K, a.ld_hidden))
    return W4A16_ERR_INVALID_SHAPE;
  if (a.ws_bytes < L->total) return W4A16_ERR_WORKSPACE_TOO_SMALL;
  if (!aligned(a.hidden, 16) || a.ld_hidden % 8 != 0) return W4A16_ERR_MISALIGNED;
  if (!aligned(a.w13, 16) || !aligned(a.w2, 16)) return W4A16_ERR_MISALIGNED;
  if (!aligned(a.s13, 2) || !aligned(a.s2, 2) || !aligned(a.out, 2))
    return W4A16_ERR_MISALIGNED;
  if (!aligned(a.topk_w, 4) || !aligned(a.ids, 4) || !aligned(a.ws, kWsAlign))
    return W4A16_ERR_MISALIGNED;
  return W4A16_OK;
}

// Workspace pointers of one call.
struct Work {
  int32_t* header;
  int32_t* sorted;
  int32_t* eids;
  int32_t* offsets;
  uint16_t* inter;
  void* partial;
  int4* tiles;
  int32_t* gemv_blocks;
  int32_t* chunks;
};

Work work_of(const Layout& L, void* ws_base) {
  char* ws = static_cast<char*>(ws_base);
  Work w;
  w.header = reinterpret_cast<int32_t*>(ws + L.off[W4A16_WS_HEADER]);
  w.sorted = reinterpret_cast<int32_t*>(ws + L.off[W4A16_WS_SORTED_IDS]);
  w.eids = reinterpret_cast<int32_t*>(ws + L.off[W4A16_WS_EXPERT_IDS]);
  w.offsets = reinterpret_cast<int32_t*>(ws + L.off[W4A16_WS_OFFSETS]);
  w.inter = reinterpret_cast<uint16_t*>(ws + L.off[W4A16_WS_INTER]);
  w.partial = ws + L.off[W4A16_WS_PARTIAL];
  w.tiles = reinterpret_cast<int4*>(ws + L.off[W4A16_WS_TILES]);
  w.gemv_blocks = reinterpret_cast<int32_t*>(ws + L.off[W4A16_WS_GEMV_BLOCKS]);
  w.chunks = L.chunked ? reinterpret_cast<int32_t*>(ws + L.off_chunks) : nullptr;
  return w;
}

// The GEMV launch of GEMM `mode` (0: w13, 1: w2).
GemvLaunch gemv_args(const FusedArgs& a, const Layout& L, const Work& w, int mode) {
  GemvLaunch g{};
  g.block_list = L.mfma ? w.gemv_blocks : nullptr;
  g.sorted = w.sorted;
  g.expert_ids = w.eids;
  g.header = w.header;
  g.n_tok = (int32_t)(a.M * a.topk);
  g.topk = (int32_t)a.topk;
  g.block = W4A16_FUSED_BLOCK_M;
  g.group = (int32_t)a.group;
  g.max_blocks = (int32_t)L.max_gemv;
  g.num_experts = (int32_t)a.E;
  g.tc = L.tc;
  g.upw = L.upw;
  g.lpr = L.lpr;
  if (L.route) {
    g.ids = a.ids;
    g.max_items = (int32_t)L.max_items;
    g.dropped_out = w.header + 1;
    // the item -> expert list of the w13 launch for the w2 launch, in the
    // sorted-ids region, which no self-routed call uses (EM >= n_tok)
    g.route_items = w.sorted;
  }
  if (mode == 0) {
    g.act = static_cast<const uint16_t*>(a.hidden);
    g.ld_act = a.ld_hidden;
    g.w = static_cast<const uint32_t*>(a.w13);
    g.s = static_cast<const uint16_t*>(a.s13);
    g.topk_w = nullptr;
    g.out = w.inter;
    g.n_out = (int32_t)a.N;
    g.kdim = (int32_t)a.K;
  } else {
    g.act = w.inter;
    g.ld_act = a.N;
    g.w = static_cast<const uint32_t*>(a.w2);
    g.s = static_cast<const uint16_t*>(a.s2);
    g.topk_w = a.topk_w;
    g.out = w.partial;
    g.partial_bf16 = L.partial_bf16;
    g.n_out = (int32_t)a.K;
    g.kdim = (int32_t)a.N;
  }
  return g;
}

// The MFMA launch of GEMM `mode`.
MfmaLaunch mfma_args(const FusedArgs& a, const Layout& L, const Work& w, int mode) {
  MfmaLaunch m{};
  m.sorted = w.sorted;
  m.tiles = w.tiles;
  m.header = w.header;
  m.n_tok = (int32_t)(a.M * a.topk);
  m.topk = (int32_t)a.topk;
  m.group = (int32_t)a.group;
  m.max_tiles = (int32_t)L.max_tiles;
  m.tile_m = L.tile_m;
  // The kernels count row tiles of their geometry's height.
  const int row_scale = L.tile_m <= kMfmaTileMSmall ? kMfmaTileN / kMfmaTileNSmall : 1;
  if (mode == 0) {
    m.act = static_cast<const uint16_t*>(a.hidden);
    m.ld_act = a.ld_hidden;
    m.w = static_cast<const uint32_t*>(a.w13);
    m.s = static_cast<const uint16_t*>(a.s13);
    m.topk_w = nullptr;
    m.out = w.inter;
    m.n_out = (int32_t)a.N;
    m.kdim = (int32_t)a.K;
    m.row_tiles = L.row_tiles_w13 * row_scale;
  } else {
    m.act = w.inter;
    m.ld_act = a.N;
    m.w = static_cast<const uint32_t*>(a.w2);
    m.s = static_cast<const uint16_t*>(a.s2);
    m.topk_w = a.topk_w;
    m.out = w.partial;
    m.partial_bf16 = L.partial_bf16;
    m.n_out = (int32_t)a.K;
    m.kdim = (int32_t)a.N;
    m.row_tiles = L.row_tiles_w2 * row_scale;
  }
  return m;
}

// Whether GEMM `mode` of the split dispatch (GEMV and MFMA work items both)
// runs as one mixed launch.
bool mixed_launch(const FusedArgs& a, const Layout& L, const Work& w, int mode) {
  return kMixedLaunches && L.gemv && L.mfma && !L.route &&
         mixed_fits(mode, mfma_args(a, L, w, mode), gemv_args(a, L, w, mode));
}

// Launch the four stages (or only stage `only` when it is 0..3); `ev`
// (5 events or null) brackets them.
int run_fused(const FusedArgs& a, const Layout& L, hipStream_t stream, hipEvent_t* ev,
              int only = -1) {
  auto want = [only](int stage) { return only < 0 || only == stage; };
  const Work w = work_of(L, a.ws);
  const int32_t n_tok = (int32_t)(a.M * a.topk);

  (void)hipGetLastError();
  if (ev && hipEventRecord(ev[0], stream) != hipSuccess) return W4A16_ERR_HIP;

  AlignLaunch al{};
  al.ids = a.ids;
  al.n_tok = n_tok;
  al.num_experts = (int32_t)a.E;
  al.block = W4A16_FUSED_BLOCK_M;
  al.em = (int32_t)L.em;
  al.n_blocks = (int32_t)L.nb;
  al.sorted = w.sorted;
  al.expert_ids = w.eids;
  al.num_post = w.header;
  al.offsets = w.offsets;
  al.dropped = w.header + 1;
  al.chunk_scratch = w.chunks;
  if (L.mfma) {
    al.tiles = w.tiles;
    al.n_tiles = w.header + 2;
    al.gemv_blocks = w.gemv_blocks;
    al.n_gemv = w.header + 3;
    al.gemv_max_tokens = L.gemv_max_tokens;
    al.tile_m = L.tile_m;
  }
  if (want(0) && !L.route && launch_align(al, stream) != hipSuccess) return W4A16_ERR_HIP;
  if (ev && hipEventRecord(ev[1], stream) != hipSuccess) return W4A16_ERR_HIP;

  // w13 (+ SiLU * up): GEMV and/or MFMA work items, in one launch where the
  // split dispatch has a mixed kernel for the shapes.
  if (want(1)) {
    const GemvLaunch g = gemv_args(a, L, w, 0);
    const MfmaLaunch m = mfma_args(a, L, w, 0);
    if (mixed_launch(a, L, w, 0)) {
      if (launch_w13_mixed(m, g, stream) != hipSuccess) return W4A16_ERR_HIP;
    } else {
      if (L.gemv && launch_w13_gemv(g, stream) != hipSuccess) return W4A16_ERR_HIP;
      if (L.mfma && launch_w13_mfma(m, stream) != hipSuccess) return W4A16_ERR_HIP;
    }
  }
  if (ev && hipEventRecord(ev[2], stream) != hipSuccess) return W4A16_ERR_HIP;

  // w2 (x routing weight): the one-launch w2 + top-k sum of few-token calls,
  // else GEMV and/or MFMA work items writing partial rows.
  if (want(2)) {
    const GemvLaunch g = gemv_args(a, L, w, 1);
    const MfmaLaunch m = mfma_args(a, L, w, 1);
    if (L.token) {
      if (launch_w2_token(g, static_cast<uint16_t*>(a.out), a.ld_out, stream) != hipSuccess)
        return W4A16_ERR_HIP;
    } else if (mixed_launch(a, L, w, 1)) {
      if (launch_w2_mixed(m, g, stream) != hipSuccess) return W4A16_ERR_HIP;
    } else {
      if (L.gemv && launch_w2_gemv(g, stream) != hipSuccess) return W4A16_ERR_HIP;
      if (L.mfma && launch_w2_mfma(m, stream) != hipSuccess) return W4A16_ERR_HIP;
    }
  }
  if (ev && hipEventRecord(ev[3], stream) != hipSuccess) return W4A16_ERR_HIP;

  CombineLaunch c{};
  c.partial = w.partial;
  c.partial_bf16 = L.partial_bf16;
  c.ids = a.ids;
  c.out = static_cast<uint16_t*>(a.out);
  c.ld_out = a.ld_out;
  c.M = (int32_t)a.M;
  c.topk = (int32_t)a.topk;
  c.K = (int32_t)a.K;
  c.num_experts = (int32_t)a.E;
  if (want(3) && !L.token && launch_combine(c, stream) != hipSuccess) return W4A16_ERR_HIP;
  if (ev && hipEventRecord(ev[4], stream) != hipSuccess) return W4A16_ERR_HIP;
  return W4A16_OK;
}

// ---- the allocation-free entry point's static scratch ----------------------
// The workspace of w4a16_moe_fused_experts_noalloc: a file-scope device array
// (each device holds its own copy, at its own address, until the process
// ends).  In host code `scratch` names a host-side stand-in, never a device
// address: the device address comes from hipGetSymbolAddress, once per device
// with that device current, and only that pointer is handed to kernels.
// Nothing in the workspace needs to start at zero (every call writes what it
// reads), so the array is never cleared.
constexpr size_t kNoallocScratchBytes = W4A16_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch's device address on `stream`'s device, which must be the
// current device (hipGetSymbolAddress resolves the current device's copy).
int scratch_for(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return W4A16_ERR_HIP;
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) return W4A16_ERR_HIP;
    if (sdev != dev) return W4A16_ERR_WRONG_DEVICE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return W4A16_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return W4A16_OK;
}

}  // namespace

extern "C" {

int w4a16_moe_abi_version(void) { return 1; }

const char* w4a16_moe_strerror(int status) {
  switch (status) {
    case W4A16_OK: return "ok";
    case W4A16_ERR_NULL_POINTER: return "a required pointer is NULL";
    case W4A16_ERR_INVALID_SHAPE: return "invalid or unsupported shape";
    case W4A16_ERR_UNSUPPORTED_GROUP:
      return "group_size must be 32, 64 or 128 and divide K and N";
    case W4A16_ERR_WORKSPACE_TOO_SMALL: return "workspace too small";
    case W4A16_ERR_MISALIGNED: return "pointer or row stride misaligned";
    case W4A16_ERR_INVALID_BLOCK: return "invalid block_size";
    case W4A16_ERR_HIP: return "HIP runtime error";
    case W4A16_ERR_UNSUPPORTED_DTYPE: return "unsupported logits dtype";
    case W4A16_ERR_INVALID_TUNING: return "invalid tuning value";
    case W4A16_ERR_SCRATCH_TOO_SMALL:
      return "call needs more workspace than the static scratch of the allocation-free "
             "entry point holds";
    case W4A16_ERR_WRONG_DEVICE:
      return "the stream's device is not the current device";
    default: return "unknown status";
  }
}

int w4a16_moe_align_sizes(int64_t M, int64_t topk, int64_t num_experts,
                          int64_t block_size, int64_t* max_num_tokens_padded,
                          int64_t* max_num_m_blocks) {
  if (!max_num_tokens_padded || !max_num_m_blocks) return W4A16_ERR_NULL_POINTER;
  return align_sizes(M, topk, num_experts, block_size, max_num_tokens_padded,
                     max_num_m_blocks);
}

int w4a16_moe_align_block_size(const int32_t* topk_ids, int64_t M, int64_t topk,
                               int64_t num_experts, int64_t block_size,
                               int32_t* sorted_token_ids, int32_t* expert_ids,
                               int32_t* num_tokens_post_padded,
                               int32_t* expert_offsets, int32_t* dropped,
                               void* stream) {
  int64_t em = 0, nb = 0;
  const int st = align_sizes(M, topk, num_experts, block_size, &em, &nb);
  if (st) return st;
  // zero-length outputs (M = 0 with block 1) may be NULL
  if ((M > 0 && !topk_ids) || (em > 0 && !sorted_token_ids) || (nb > 0 && !expert_ids) ||
      !num_tokens_post_padded)
    return W4A16_ERR_NULL_POINTER;
  AlignLaunch al{};
  al.ids = topk_ids;
  al.n_tok = (int32_t)(M * topk);
  al.num_experts = (int32_t)num_experts;
  al.block = (int32_t)block_size;
  al.em = (int32_t)em;
  al.n_blocks = (int32_t)nb;
  al.sorted = sorted_token_ids;
  al.expert_ids = expert_ids;
  al.num_post = num_tokens_post_padded;
  al.offsets = expert_offsets;
  al.dropped = dropped;
  (void)hipGetLastError();
  return launch_align(al, static_cast<hipStream_t>(stream)) == hipSuccess ? W4A16_OK
                                                                         : W4A16_ERR_HIP;
}

int w4a16_moe_default_tuning(int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                             int64_t K, int64_t group_size, w4a16_moe_tuning* tuning) {
  if (!tuning) return W4A16_ERR_NULL_POINTER;
  Layout L;
  const Tuning T = default_tuning();
  const int st = compute_layout(M, topk, num_experts, N, K, group_size, T, &L);
  if (st) return st;
  *tuning = w4a16_moe_tuning{};
  tuning->gemv_only_max_m = T.gemv_only_max_m;
  tuning->gemv_max_tokens = L.gemv_max_tokens;
  tuning->gemv_tokens_per_pass = T.tc;
  tuning->mfma_tile_m = L.tile_m;
  tuning->gemv_units_per_wg = T.upw;
  tuning->gemv_lanes_per_row = T.lpr;
  tuning->w2_fused_max_m = T.w2_fused_max_m;
  return W4A16_OK;
}

int w4a16_moe_workspace_size_ex(int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                                int64_t K, int64_t group_size,
                                const w4a16_moe_tuning* tuning, size_t* bytes) {
  if (!bytes) return W4A16_ERR_NULL_POINTER;
  Tuning T;
  int st = resolve_tuning(tuning, &T);
  if (st) return st;
  Layout L;
  st = compute_layout(M, topk, num_experts, N, K, group_size, T, &L);
  if (st) return st;
  *bytes = L.total;
  return W4A16_OK;
}

int w4a16_moe_workspace_size(int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                             int64_t K, int64_t group_size, size_t* bytes) {
  return w4a16_moe_workspace_size_ex(M, topk, num_experts, N, K, group_size, nullptr,
                                     bytes);
}

int w4a16_moe_workspace_layout_ex(int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                                  int64_t K, int64_t group_size,
                                  const w4a16_moe_tuning* tuning,
                                  size_t offsets[W4A16_WS_NFIELDS]) {
  if (!offsets) return W4A16_ERR_NULL_POINTER;
  Tuning T;
  int st = resolve_tuning(tuning, &T);
  if (st) return st;
  Layout L;
  st = compute_layout(M, topk, num_experts, N, K, group_size, T, &L);
  if (st) return st;
  for (int i = 0; i < W4A16_WS_NFIELDS; ++i) offsets[i] = L.off[i];
  return W4A16_OK;
}

int w4a16_moe_workspace_layout(int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                               int64_t K, int64_t group_size,
                               size_t offsets[W4A16_WS_NFIELDS]) {
  return w4a16_moe_workspace_layout_ex(M, topk, num_experts, N, K, group_size, nullptr,
                                       offsets);
}

int w4a16_moe_stage_launches(int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                             int64_t K, int64_t group_size, const w4a16_moe_tuning* tuning,
                             int32_t launches[4]) {
  if (!launches) return W4A16_ERR_NULL_POINTER;
  Tuning T;
  int st = resolve_tuning(tuning, &T);
  if (st) return st;
  Layout L;
  st = compute_layout(M, topk, num_experts, N, K, group_size, T, &L);
  if (st) return st;
  for (int i = 0; i < 4; ++i) launches[i] = 0;
  if (M == 0) return W4A16_OK;
  // The same decisions as run_fused (scales assumed 16-byte aligned, as
  // torch allocations are).
  // Stand-in pointers, suitably aligned: only the mixed-launch decision
  // reads them (scale alignment).
  alignas(256) static const unsigned char stand_in[256] = {};
  const void* p = stand_in;
  const FusedArgs a{p, K, p, p, p, p, reinterpret_cast<const float*>(p),
                    reinterpret_cast<const int32_t*>(p), M, topk, num_experts, N, K,
                    group_size, const_cast<void*>(p), K, const_cast<void*>(p), L.total, tuning};
  const Work w = work_of(L, const_cast<void*>(p));
  auto gemm = [&](int mode) {
    return mixed_launch(a, L, w, mode) ? 1 : (L.gemv ? 1 : 0) + (L.mfma ? 1 : 0);
  };
  launches[0] = L.route ? 0 : (L.chunked ? 2 : 1);
  launches[1] = gemm(0);
  launches[2] = L.token ? 1 : gemm(1);
  launches[3] = L.token ? 0 : 1;
  return W4A16_OK;
}

int w4a16_moe_fused_experts_ex(const void* hidden, int64_t ld_hidden,
                               const void* w13_packed, const void* w2_packed,
                               const void* w13_scale, const void* w2_scale,
                               const float* topk_weights, const int32_t* topk_ids,
                               int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                               int64_t K, int64_t group_size, void* out, int64_t ld_out,
                               void* workspace, size_t workspace_bytes, void* stream,
                               const w4a16_moe_tuning* tuning) {
  const FusedArgs a{hidden, ld_hidden, w13_packed, w2_packed, w13_scale, w2_scale,
                    topk_weights, topk_ids, M, topk, num_experts, N, K, group_size,
                    out, ld_out, workspace, workspace_bytes, tuning};
  Layout L;
  const int st = validate(a, &L);
  if (st || M == 0) return st;
  return run_fused(a, L, static_cast<hipStream_t>(stream), nullptr);
}

int w4a16_moe_fused_experts(const void* hidden, int64_t ld_hidden, const void* w13_packed,
                            const void* w2_packed, const void* w13_scale,
                            const void* w2_scale, const float* topk_weights,
                            const int32_t* topk_ids, int64_t M, int64_t topk,
                            int64_t num_experts, int64_t N, int64_t K, int64_t group_size,
                            void* out, int64_t ld_out, void* workspace,
                            size_t workspace_bytes, void* stream) {
  return w4a16_moe_fused_experts_ex(hidden, ld_hidden, w13_packed, w2_packed, w13_scale,
                                    w2_scale, topk_weights, topk_ids, M, topk, num_experts,
                                    N, K, group_size, out, ld_out, workspace,
                                    workspace_bytes, stream, nullptr);
}

int w4a16_moe_fused_experts_profiled(
    const void* hidden, int64_t ld_hidden, const void* w13_packed, const void* w2_packed,
    const void* w13_scale, const void* w2_scale, const float* topk_weights,
    const int32_t* topk_ids, int64_t M, int64_t topk, int64_t num_experts, int64_t N,
    int64_t K, int64_t group_size, void* out, int64_t ld_out, void* workspace,
    size_t workspace_bytes, void* stream, float stage_ms[4]) {
  if (!stage_ms) return W4A16_ERR_NULL_POINTER;
  const FusedArgs a{hidden, ld_hidden, w13_packed, w2_packed, w13_scale, w2_scale,
                    topk_weights, topk_ids, M, topk, num_experts, N, K, group_size,
                    out, ld_out, workspace, workspace_bytes, nullptr};
  Layout L;
  int st = validate(a, &L);
  if (st) return st;
  for (int i = 0; i < 4; ++i) stage_ms[i] = 0.0f;
  if (M == 0) return W4A16_OK;
  hipEvent_t ev[5];
  int made = 0;
  for (; made < 5; ++made)
    if (hipEventCreate(&ev[made]) != hipSuccess) break;
  if (made < 5) {
    for (int i = 0; i < made; ++i) (void)hipEventDestroy(ev[i]);
    return W4A16_ERR_HIP;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = run_fused(a, L, s, ev);
  if (st == W4A16_OK && hipEventSynchronize(ev[4]) != hipSuccess) st = W4A16_ERR_HIP;
  if (st == W4A16_OK) {
    for (int i = 0; i < 4; ++i) {
      float ms = 0.0f;
      if (hipEventElapsedTime(&ms, ev[i], ev[i + 1]) != hipSuccess) st = W4A16_ERR_HIP;
      stage_ms[i] = ms;
    }
  }
  for (int i = 0; i < 5; ++i) (void)hipEventDestroy(ev[i]);
  return st;
}

int w4a16_moe_run_stage_ex(int stage, const void* hidden, int64_t ld_hidden,
                           const void* w13_packed, const void* w2_packed,
                           const void* w13_scale, const void* w2_scale,
                           const float* topk_weights, const int32_t* topk_ids, int64_t M,
                           int64_t topk, int64_t num_experts, int64_t N, int64_t K,
                           int64_t group_size, void* out, int64_t ld_out, void* workspace,
                           size_t workspace_bytes, void* stream,
                           const w4a16_moe_tuning* tuning) {
  if (stage < 0 || stage > 3) return W4A16_ERR_INVALID_SHAPE;
  const FusedArgs a{hidden, ld_hidden, w13_packed, w2_packed, w13_scale, w2_scale,
                    topk_weights, topk_ids, M, topk, num_experts, N, K, group_size,
                    out, ld_out, workspace, workspace_bytes, tuning};
  Layout L;
  const int st = validate(a, &L);
  if (st || M == 0) return st;
  return run_fused(a, L, static_cast<hipStream_t>(stream), nullptr, stage);
}

int w4a16_moe_run_stage(int stage, const void* hidden, int64_t ld_hidden,
                        const void* w13_packed, const void* w2_packed,
                        const void* w13_scale, const void* w2_scale,
                        const float* topk_weights, const int32_t* topk_ids, int64_t M,
                        int64_t topk, int64_t num_experts, int64_t N, int64_t K,
                        int64_t group_size, void* out, int64_t ld_out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return w4a16_moe_run_stage_ex(stage, hidden, ld_hidden, w13_packed, w2_packed, w13_scale,
                                w2_scale, topk_weights, topk_ids, M, topk, num_experts, N,
                                K, group_size, out, ld_out, workspace, workspace_bytes,
                                stream, nullptr);
}

int w4a16_moe_fused_experts_noalloc(const void* hidden, int64_t ld_hidden,
                                    const void* w13_packed, const void* w2_packed,
                                    const void* w13_scale, const void* w2_scale,
                                    const float* topk_weights, const int32_t* topk_ids,
                                    int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                                    int64_t K, int64_t group_size, void* out, int64_t ld_out,
                                    void* stream, const w4a16_moe_tuning* tuning) {
  // The size check comes first: it needs no device and rejects a call too
  // big for the scratch before anything else runs.  The layout is the one
  // validate() builds for these pointers (the MFMA kernels need 16-byte
  // aligned scales; without them every expert runs on the GEMV kernels,
  // whose work lists are sized differently).
  Tuning T;
  int st = resolve_tuning(tuning, &T);
  if (st) return st;
  Layout L;
  st = compute_layout(M, topk, num_experts, N, K, group_size, T, &L,
                      aligned(w13_scale, 16) && aligned(w2_scale, 16));
  if (st) return st;
  if (M == 0) return W4A16_OK;
  if (L.total > kNoallocScratchBytes) return W4A16_ERR_SCRATCH_TOO_SMALL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  st = scratch_for(s, &ws);
  if (st) return st;
  const FusedArgs a{hidden, ld_hidden, w13_packed, w2_packed, w13_scale, w2_scale,
                    topk_weights, topk_ids, M, topk, num_experts, N, K, group_size,
                    out, ld_out, ws, kNoallocScratchBytes, tuning};
  st = validate(a, &L);
  if (st == W4A16_ERR_WORKSPACE_TOO_SMALL) return W4A16_ERR_SCRATCH_TOO_SMALL;
  if (st) return st;
  return run_fused(a, L, s, nullptr);
}

int w4a16_moe_capture_id(void* stream, uint64_t* capture_id) {
  if (!capture_id) return W4A16_ERR_NULL_POINTER;
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  if (hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &status, &id) != hipSuccess)
    return W4A16_ERR_HIP;
  *capture_id = status == hipStreamCaptureStatusActive ? (uint64_t)id : 0;
  return W4A16_OK;
}

int w4a16_moe_dropped_pairs(const void* workspace, int32_t* count, void* stream) {
  if (!workspace || !count) return W4A16_ERR_NULL_POINTER;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int32_t* header = static_cast<const int32_t*>(workspace);  // header is field 0
  if (hipMemcpyAsync(count, header + 1, sizeof(int32_t), hipMemcpyDeviceToHost, s) !=
      hipSuccess)
    return W4A16_ERR_HIP;
  return hipStreamSynchronize(s) == hipSuccess ? W4A16_OK : W4A16_ERR_HIP;
}

int w4a16_moe_router_topk_softmax(const void* logits, int logits_dtype,
                                  int64_t ld_logits, int64_t M, int64_t num_experts,
                                  int64_t topk, int renormalize, float* topk_weights,
                                  int32_t* topk_ids, void* stream) {
  if (logits_dtype != W4A16_LOGITS_F32 && logits_dtype != W4A16_LOGITS_BF16)
    return W4A16_ERR_UNSUPPORTED_DTYPE;
  if (M < 0 || num_experts < 1 || num_experts > kMaxExperts) return W4A16_ERR_INVALID_SHAPE;
  if (topk < 1 || topk > W4A16_ROUTER_MAX_TOPK || topk > num_experts)
    return W4A16_ERR_INVALID_SHAPE;
  if (renormalize != 0 && renormalize != 1) return W4A16_ERR_INVALID_SHAPE;
  if (M > 0 && ld_logits < num_experts) return W4A16_ERR_INVALID_SHAPE;
  if (M > (int64_t)INT_MAX / topk) return W4A16_ERR_INVALID_SHAPE;
  if (M == 0) return W4A16_OK;
  if (!logits || !topk_weights || !topk_ids) return W4A16_ERR_NULL_POINTER;
  const uintptr_t elt = logits_dtype == W4A16_LOGITS_BF16 ? 2 : 4;
  if ((uintptr_t)logits % elt || (uintptr_t)topk_weights % 4 || (uintptr_t)topk_ids % 4)
    return W4A16_ERR_MISALIGNED;
  RouterLaunch r{};
  r.logits = logits;
  r.ld = ld_logits;
  r.M = M;
  r.E = (int32_t)num_experts;
  r.topk = (int32_t)topk;
  r.bf16 = logits_dtype == W4A16_LOGITS_BF16;
  r.renormalize = renormalize;
  r.weights = topk_weights;
  r.ids = topk_ids;
  (void)hipGetLastError();
  return launch_router(r, static_cast<hipStream_t>(stream)) == hipSuccess ? W4A16_OK
                                                                         : W4A16_ERR_HIP;
}

}  // extern "C"
