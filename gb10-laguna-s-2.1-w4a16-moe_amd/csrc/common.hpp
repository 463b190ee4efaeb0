// Shared device helpers and the host-side launcher declarations of the
// W4A16 MoE library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace w4a16 {

constexpr int kWave = 64;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 (hardware conversion on gfx950).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  __bf16 h = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// DPP lane moves on 32-bit values.  All controls used here read a valid lane
// for every destination lane.
//   0xB1  quad_perm [1,0,3,2]  (lane ^ 1)
//   0x4E  quad_perm [2,3,0,1]  (lane ^ 2)
//   0x141 row_half_mirror      (lane i <- lane 7-i within 8 lanes)
//   0x140 row_mirror           (lane i <- lane 15-i within 16 lanes)
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of 4 lanes; every lane of the quad gets the sum.
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  return v;
}

// Sum over aligned groups of 8 lanes; every lane of the group gets the sum.
__device__ __forceinline__ float oct_sum(float v) {
  v = quad_sum(v);
  v += dpp_f32<0x141>(v);
  return v;
}

__device__ __forceinline__ uint64_t ballot(bool p) {
  return __builtin_amdgcn_ballot_w64(p);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const uint32_t lane = __lane_id();
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Exclusive scan of one int per thread over a workgroup of NT threads
// (NT <= 1024); wave_tot is LDS scratch of 17 ints.  All threads must call.
template <int NT>
__device__ __forceinline__ int wg_exclusive_scan(int v, int* wave_tot, int* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) wave_tot[wid] = x;
  __syncthreads();
  if (wid == 0) {
    const int t = lane < NW ? wave_tot[lane] : 0;
    int s = t;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(s, d, 64);
      if (lane >= d) s += y;
    }
    if (lane < NW) wave_tot[lane] = s - t;
    if (lane == NW - 1) wave_tot[16] = s;
  }
  __syncthreads();
  *total = wave_tot[16];
  const int excl = x - v + wave_tot[wid];
  __syncthreads();
  return excl;
}

}  // namespace w4a16

// ---- host launchers (defined next to their kernels) ----------------------
namespace w4a16 {

// MFMA tile: token slots x weight rows of one workgroup.  An expert's pairs
// are cut into the fewest tiles of at most tile_m slots (64, 128 or 192,
// chosen per call), of near-equal size.  Tiles of at most 64 slots run on
// 4-wave workgroups of 128-row row tiles, the others on 8-wave workgroups of
// 256-row row tiles.
constexpr int kMfmaTileMSmall = 64;
constexpr int kMfmaTileMMin = 128;
constexpr int kMfmaTileMMax = 192;
constexpr int kMfmaTileN = 256;
constexpr int kMfmaTileNSmall = 128;

struct AlignLaunch {
  const int32_t* ids;
  int32_t n_tok;
  int32_t num_experts;
  int32_t block;
  int32_t em;        // sorted_token_ids length
  int32_t n_blocks;  // expert_ids length
  int32_t* sorted;
  int32_t* expert_ids;
  int32_t* num_post;
  int32_t* offsets;  // may be null, [E+1]
  int32_t* dropped;  // may be null, [1]
  // Work lists of the fused call (all null for the plain sort).  Experts
  // with more than gemv_max_tokens pairs get ceil(count / tile_m) MFMA tiles
  // of near-equal size (multiples of 32 slots but the last); the others keep
  // their single sorted block on the GEMV path.
  // Requires gemv_max_tokens < block.
  int4* tiles;           // [max tiles] (expert, first slot, count, 0)
  int32_t* n_tiles;      // [1]
  int32_t* gemv_blocks;  // [max blocks] block indices, ascending
  int32_t* n_gemv;       // [1]
  int32_t gemv_max_tokens;
  int32_t tile_m;        // MFMA tile height (slots)
  // Optional scratch of align_chunk_scratch_ints(n_tok, E) int32: with it,
  // batches of at least kAlignChunkedMinPairs pairs sort in chunks over many
  // workgroups (two launches) instead of one workgroup.
  int32_t* chunk_scratch;
};
constexpr int kAlignChunkedMinPairs = 8192;
constexpr int kAlignChunkedMaxE = 512;
int align_chunks(int n_tok);
inline size_t align_chunk_scratch_ints(int n_tok, int num_experts) {
  return (size_t)align_chunks(n_tok) * (num_experts + 1);
}
hipError_t launch_align(const AlignLaunch& a, hipStream_t stream);

struct GemvLaunch {
  const uint16_t* act;     // bf16 activation rows
  int64_t ld_act;          // row stride (elements)
  const uint32_t* w;       // packed weights [E, rows_total, kdim/8]
  const uint16_t* s;       // bf16 scales   [E, rows_total, kdim/G]
  const int32_t* sorted;
  const int32_t* expert_ids;
  const int32_t* header;   // [0] = num_tokens_post_padded
  const float* topk_w;     // w2 only
  void* out;               // w13: bf16 inter [n_tok, n_out]; w2: partial [n_tok, n_out]
  int32_t partial_bf16;    // w2: partial rows are bf16 (else fp32)
  int32_t n_tok;
  int32_t topk;
  int32_t block;
  int32_t n_out;           // output rows (N for w13, K for w2)
  int32_t kdim;            // reduction length (K for w13, N for w2)
  int32_t group;
  int32_t max_blocks;      // upper bound of active blocks
  int32_t num_experts;
  const int32_t* block_list;  // null: work item b is block b; else blocks
                              // block_list[0 .. header[3])
  uint32_t nib_mask;          // set by the launcher (see gemv.hip)
  uint32_t nib_magic;
  // Self-routing (small batches, the align kernel is not run): when `ids`
  // is set, work item i is flat slot i, which works when it is the first
  // slot routed to its expert, found by every wave from topk_ids itself.
  const int32_t* ids;      // [n_tok] topk_ids
  int32_t max_items;       // work items: n_tok
  int32_t* dropped_out;    // w13: [1] pairs with ids outside [0, E)
  int32_t tc;              // token rows per pass: 0 = chosen by the launcher,
                           // else 1, 2 or 4 (lowered while LDS does not fit)
  int32_t upw;             // row slabs per workgroup: 0 = chosen by the
                           // launcher, else 1, 2 or 4 (1 for run-time loops)
  int32_t lpr;             // lanes per weight row: 0 = chosen by the launcher,
                           // else 8 or 32 (32 for passes of at most 2 tokens)
  // Self-routing: the expert of every work item (-1: none), [max_items];
  // written by the w13 launch, read by the w2 launch.  Null: each launch
  // routes on its own.
  int32_t* route_items;
};
hipError_t launch_w13_gemv(const GemvLaunch& a, hipStream_t stream);
hipError_t launch_w2_gemv(const GemvLaunch& a, hipStream_t stream);
// Few-token calls: w2 and the top-k combine in one launch, writing the bf16
// output rows `out` (row stride ld_out) of the n_tok / topk tokens.
bool w2_token_fits(int topk, int K, int N);
hipError_t launch_w2_token(const GemvLaunch& a, uint16_t* out, int64_t ld_out,
                           hipStream_t stream);
// Self-routing: whether the routing tables plus one staged row fit in LDS.
bool gemv_route_fits(int n_tok, int num_experts, int K, int N);

struct MfmaLaunch {
  const uint16_t* act;     // bf16 activation rows (x for w13, inter for w2)
  int64_t ld_act;
  const uint32_t* w;       // packed weights [E, rows_total, kdim/8]
  const uint16_t* s;       // bf16 scales   [E, rows_total, kdim/G]
  const int32_t* sorted;
  const int4* tiles;       // (expert, first slot, count, 0)
  const int32_t* header;   // [2] = number of tiles
  const float* topk_w;     // w2 only
  void* out;               // w13: bf16 inter [n_tok, n_out]; w2: partial [n_tok, n_out]
  int32_t partial_bf16;    // w2: partial rows are bf16 (else fp32)
  int32_t n_tok;
  int32_t topk;
  int32_t n_out;           // N for w13 (2N weight rows), K for w2
  int32_t kdim;
  int32_t group;
  int32_t max_tiles;
  int32_t tile_m;          // token slots per tile, at most (128 or 192)
  int32_t row_tiles;       // row tiles (of the geometry's height) one workgroup runs in turn
};
hipError_t launch_w13_mfma(const MfmaLaunch& a, hipStream_t stream);
hipError_t launch_w2_mfma(const MfmaLaunch& a, hipStream_t stream);

// The split dispatch's GEMV and MFMA work items of one GEMM (mode 0: w13,
// 1: w2) in one launch, when mixed_fits(mode, m, g): m and g are the two
// launches' arguments.  The 128-row MFMA geometry (tiles of at most 64
// slots), 8-lane GEMV rows with 2 or 4 token rows per pass, one row slab per
// workgroup and the unrolled step loop of K = 3072 (w13) / N = 1024 (w2).
bool mixed_fits(int mode, const MfmaLaunch& m, const GemvLaunch& g);
hipError_t launch_w13_mixed(const MfmaLaunch& m, const GemvLaunch& g, hipStream_t stream);
hipError_t launch_w2_mixed(const MfmaLaunch& m, const GemvLaunch& g, hipStream_t stream);

struct CombineLaunch {
  const void* partial;     // [M*topk, K], bf16 or fp32
  int32_t partial_bf16;
  const int32_t* ids;      // [M, topk]
  uint16_t* out;           // bf16 [M, ld_out]
  int64_t ld_out;
  int32_t M;
  int32_t topk;
  int32_t K;
  int32_t num_experts;
};
hipError_t launch_combine(const CombineLaunch& a, hipStream_t stream);

struct RouterLaunch {
  const void* logits;  // [M, ld] fp32 or bf16
  int64_t ld;          // row stride in elements
  int64_t M;
  int32_t E;           // 1..1024
  int32_t topk;        // 1..min(64, E)
  int32_t bf16;        // logits are bf16
  int32_t renormalize; // 1: softmax over the selected logits; 0: over all E
  float* weights;      // [M, topk]
  int32_t* ids;        // [M, topk]
};
hipError_t launch_router(const RouterLaunch& a, hipStream_t stream);

}  // namespace w4a16
