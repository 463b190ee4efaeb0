/*
 * w4a16_moe.h -- C ABI of the MI355X (gfx950) W4A16 grouped-expert MoE path.
 *
 * One MoE layer: out[M,K] = sum_t w[m,t] * W2_e (SiLU(Wg_e x_m) * (Wu_e x_m)),
 * e = topk_ids[m,t], with int4 weights stored in the compressed-tensors
 * "pack-quantized" layout, consumed unchanged:
 *
 *   w13_packed  [E, 2N, K/8]  int32  (== [E, 2N, K/2] uint8), rows 0..N-1 gate,
 *                                    rows N..2N-1 up; element k of a row is
 *                                    nibble (k % 8) of word k/8, value = code-8
 *   w13_scale   [E, 2N, K/G]  bf16   one symmetric scale per G elements of K
 *   w2_packed   [E, K,  N/8]  int32
 *   w2_scale    [E, K,  N/G]  bf16
 *   hidden      [M, K]        bf16   (row stride ld_hidden elements)
 *   topk_ids    [M, topk]     int32  contiguous
 *   topk_weights[M, topk]     fp32   contiguous
 *   out         [M, K]        bf16   (row stride ld_out elements)
 *
 * Contract of every entry point:
 *   - status 0 (W4A16_OK) on success; argument errors are detected on the
 *     host before any GPU work is enqueued;
 *   - all GPU work is enqueued on `stream` (a hipStream_t; NULL = default
 *     stream) with no host synchronisation and no device allocation, so a
 *     call can be captured into a HIP graph (the *_profiled variant excepted);
 *   - the library holds no mutable global state (save the static scratch of
 *     w4a16_moe_fused_experts_noalloc); concurrent calls that share one
 *     workspace race, calls with distinct workspaces do not;
 *   - inputs are never modified.
 *
 * Expert ids outside [0, E) are not routed: the pair contributes nothing to
 * the output and is counted in the workspace's dropped-pair counter
 * (w4a16_moe_dropped_pairs).  The reference indexes out of bounds instead.
 */
#ifndef W4A16_MOE_H
#define W4A16_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define W4A16_OK                      0
#define W4A16_ERR_NULL_POINTER        1  /* a required pointer is NULL        */
#define W4A16_ERR_INVALID_SHAPE       2  /* negative / inconsistent / too big */
#define W4A16_ERR_UNSUPPORTED_GROUP   3  /* group size not 32, 64 or 128 ...   */
#define W4A16_ERR_WORKSPACE_TOO_SMALL 4
#define W4A16_ERR_MISALIGNED          5  /* pointer / row stride alignment    */
#define W4A16_ERR_INVALID_BLOCK       6  /* block_size < 1                    */
#define W4A16_ERR_HIP                 7  /* a HIP runtime call failed         */
#define W4A16_ERR_UNSUPPORTED_DTYPE   8  /* router logits not fp32 or bf16    */
#define W4A16_ERR_INVALID_TUNING      9  /* a w4a16_moe_tuning field out of range */
#define W4A16_ERR_SCRATCH_TOO_SMALL  10  /* call too big for the static scratch of
                                            w4a16_moe_fused_experts_noalloc    */
#define W4A16_ERR_WRONG_DEVICE       11  /* w4a16_moe_fused_experts_noalloc: the
                                            stream's device is not the current
                                            device                            */

/* Indices of w4a16_moe_workspace_layout()'s offsets array. */
#define W4A16_WS_SORTED_IDS   0  /* int32 [EM]            sorted token-slot ids   */
#define W4A16_WS_EXPERT_IDS   1  /* int32 [EM/16]         expert of each block    */
#define W4A16_WS_HEADER       2  /* int32 [64]: [0] num_tokens_post_padded,
                                    [1] dropped pairs, [2] MFMA tiles,
                                    [3] GEMV blocks, [4..] reserved              */
#define W4A16_WS_OFFSETS      3  /* int32 [E+1]           padded expert offsets   */
#define W4A16_WS_INTER        4  /* bf16  [M*topk, N]     SiLU(gate)*up           */
#define W4A16_WS_PARTIAL      5  /* bf16  [M*topk, K]     weighted w2 products
                                    (fp32 when M <= 4)                           */
#define W4A16_WS_TILES        6  /* int32 [tiles][4]      MFMA work list          */
#define W4A16_WS_GEMV_BLOCKS  7  /* int32 [blocks]        GEMV work list          */
#define W4A16_WS_NFIELDS      8
/* Calls with M <= W4A16_GEMV_ONLY_MAX_M skip the align kernel: the GEMV
 * kernels route themselves from topk_ids.  Those calls write only the
 * header's dropped count [1], INTER, PARTIAL (not PARTIAL when M <= 4: w2
 * and the top-k sum then run as one kernel) and, in the first M*topk entries
 * of SORTED_IDS, the w13 launch's expert of each work item (-1: none), which
 * the w2 launch reads; the other fields keep whatever they held. */

/* Token-block size the fused call uses for its internal expert sort. */
#define W4A16_FUSED_BLOCK_M 16

/* Experts with more (token, slot) pairs than this run on the MFMA kernels
 * when M > W4A16_GEMV_ONLY_MAX_M and N and K are multiples of 256; the others
 * run on the GEMV kernels. */
#define W4A16_GEMV_MAX_TOKENS 4

/* Calls with at most this many tokens run every expert on the GEMV kernels
 * (by default; see w4a16_moe_tuning): few experts then hold more than a
 * handful of pairs, and the MFMA launches would only add their fixed cost. */
#define W4A16_GEMV_ONLY_MAX_M 24

/*
 * Sizes of moe_align_block_size's outputs.
 * Replaces the buffer sizing of _align_workspace,
 * kernels/w4a16_moe.py:153-157:
 *   EM = round_up(M*topk + E*(block-1), block),  n_blocks = EM / block.
 */
int w4a16_moe_align_sizes(int64_t M, int64_t topk, int64_t num_experts,
                          int64_t block_size, int64_t* max_num_tokens_padded,
                          int64_t* max_num_m_blocks);

/*
 * Sort the M*topk (token, slot) pairs by expert, pad every expert to a
 * multiple of block_size and emit per-block expert ids.
 * Replaces moe_align_block_size, kernels/w4a16_moe.py:187-290, with
 * bit-identical outputs over the whole fixed-size buffers:
 *   sorted_token_ids[EM]  flat index f = m*topk + t, stable (ascending f)
 *                         within an expert; padding slots hold M*topk;
 *   expert_ids[EM/block]  expert of each block, -1 after the padded end;
 *   num_tokens_post_padded[1].
 * Optional outputs (may be NULL): expert_offsets[E+1] (exclusive prefix of
 * padded counts) and dropped[1] (pairs whose id is outside [0, E)).
 * One kernel launch on `stream`.
 */
int w4a16_moe_align_block_size(const int32_t* topk_ids, int64_t M,
                               int64_t topk, int64_t num_experts,
                               int64_t block_size, int32_t* sorted_token_ids,
                               int32_t* expert_ids,
                               int32_t* num_tokens_post_padded,
                               int32_t* expert_offsets, int32_t* dropped,
                               void* stream);

/*
 * Device scratch needed by w4a16_moe_fused_experts (bytes, 256-aligned).
 * Replaces the scratch pools _align_workspace / _gemm_workspace,
 * kernels/w4a16_moe.py:141-184 and :293-316.
 */
int w4a16_moe_workspace_size(int64_t M, int64_t topk, int64_t num_experts,
                             int64_t N, int64_t K, int64_t group_size,
                             size_t* bytes);

/* Byte offsets of the workspace's fields (W4A16_WS_*), for inspection. */
int w4a16_moe_workspace_layout(int64_t M, int64_t topk, int64_t num_experts,
                               int64_t N, int64_t K, int64_t group_size,
                               size_t offsets[W4A16_WS_NFIELDS]);

/*
 * The fused W4A16 MoE layer.
 * Replaces fused_experts_w4a16, kernels/w4a16_moe.py:678-909 (expert sort,
 * w13 dequant-GEMM with SiLU(gate)*up, w2 dequant-GEMM with the top-k
 * weighted combine).  Weights are the unchanged pack-quantized tensors (no
 * repack).  Accumulation is fp32; the rounding points are the reference's:
 * the w13 output (SiLU(gate)*up) is rounded to bf16, and so is each
 * top-k-weighted w2 row when M > 4 (the reference's bf16 partial buffer,
 * :311; at M <= 4 the rows stay fp32, as in its fp32 atomic path, :763).
 * The top-k combine is summed in fp32 in slot order (deterministic).
 * Requirements: K and N multiples of 32 and of group_size, at most 16384;
 * group_size in {32, 64, 128}; 1 <= topk <= 256; 1 <= E <= 1024;
 * M * topk < 2^30; hidden and packed-weight pointers 16-byte aligned;
 * ld_hidden % 8 == 0; workspace 256-byte aligned and at least
 * w4a16_moe_workspace_size bytes.  Calls that run the MFMA kernels (M above
 * the GEMV-only bound, N and K multiples of 256) address activation and
 * output rows with 32-bit byte offsets: they also need M * ld_hidden * 2,
 * M * topk * N * 2 and M * topk * K * 2 (* 4 when M <= 4) at most
 * 2^32 - 4097 bytes (W4A16_ERR_INVALID_SHAPE otherwise, before any GPU
 * work); at K = 3072, topk = 10 that is M <= 69,904.
 */
int w4a16_moe_fused_experts(const void* hidden, int64_t ld_hidden,
                            const void* w13_packed, const void* w2_packed,
                            const void* w13_scale, const void* w2_scale,
                            const float* topk_weights, const int32_t* topk_ids,
                            int64_t M, int64_t topk, int64_t num_experts,
                            int64_t N, int64_t K, int64_t group_size,
                            void* out, int64_t ld_out, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Same computation as w4a16_moe_fused_experts, with HIP events recorded
 * between its stages; waits for the stream and writes each stage's device
 * time in milliseconds to stage_ms[4] = {align, w13, w2, combine}.
 * Measurement helper: no counterpart in the reference.
 */
int w4a16_moe_fused_experts_profiled(
    const void* hidden, int64_t ld_hidden, const void* w13_packed,
    const void* w2_packed, const void* w13_scale, const void* w2_scale,
    const float* topk_weights, const int32_t* topk_ids, int64_t M,
    int64_t topk, int64_t num_experts, int64_t N, int64_t K,
    int64_t group_size, void* out, int64_t ld_out, void* workspace,
    size_t workspace_bytes, void* stream, float stage_ms[4]);

/*
 * Launch a single stage of w4a16_moe_fused_experts on `stream`:
 * 0 = expert sort, 1 = w13 + SiLU*up, 2 = w2 + routing weight, 3 = combine.
 * Each stage reads what the previous stages left in `workspace`, so a full
 * call with the same arguments and workspace must have run first.  Lets a
 * benchmark time one kernel in isolation; no counterpart in the reference.
 */
int w4a16_moe_run_stage(int stage, const void* hidden, int64_t ld_hidden,
                        const void* w13_packed, const void* w2_packed,
                        const void* w13_scale, const void* w2_scale,
                        const float* topk_weights, const int32_t* topk_ids,
                        int64_t M, int64_t topk, int64_t num_experts, int64_t N,
                        int64_t K, int64_t group_size, void* out, int64_t ld_out,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * The capture sequence of `stream`: *capture_id = 0 when the stream is not
 * being captured into a HIP graph, else the runtime's id of the capture in
 * progress (hipStreamGetCaptureInfo).  Lets a host-side workspace pool give
 * each captured graph its own workspace.  No GPU work, no synchronisation.
 * Host helper; no counterpart in the reference, which pools its scratch per
 * shape (kernels/w4a16_moe.py:293-316).
 */
int w4a16_moe_capture_id(void* stream, uint64_t* capture_id);

/*
 * Read the dropped-pair counter the last fused call left in `workspace`
 * (waits for `stream`).  No counterpart in the reference, which has no range
 * check on topk_ids.
 */
int w4a16_moe_dropped_pairs(const void* workspace, int32_t* count,
                            void* stream);

/* ---- allocation-free variant -------------------------------------------- */
/* Bytes of the library's static device scratch (per device). */
#define W4A16_NOALLOC_SCRATCH_BYTES (64u << 20)

/* ---- dispatch tuning (the per-M tile selector) -------------------------- */
/*
 * How a call splits its work between the kernels.  The analogue of the
 * reference's tuned per-M kernel configurations: its fused_experts_w4a16
 * takes block_m/block_n/block_k (kernels/w4a16_moe.py:678-690) and the stock
 * path reads them from a per-device JSON keyed by M
 * (configs/E=256,N=1024,device_name=NVIDIA_GB10,dtype=int4_w4a16.json,
 * written by bench/tune_configs.py).  Here the tile shapes are fixed per
 * kernel and the choices are which kernels run:
 *   gemv_only_max_m       calls with M <= this run every expert on the GEMV
 *                         kernels (routing themselves when it fits in LDS);
 *   gemv_max_tokens       larger calls (N, K multiples of 256) send experts
 *                         with more (token, slot) pairs than this (0..15) to
 *                         the MFMA kernels, the others to the GEMV kernels;
 *                         0 sends every expert to the MFMA kernels and skips
 *                         the GEMV launches (the built-in choice once experts
 *                         average 32 or more pairs, 4 below that);
 *   gemv_tokens_per_pass  token rows one GEMV pass reads the weights for:
 *                         0 (the library's choice), 1, 2 or 4;
 *   mfma_tile_m           most (token, slot) pairs of one expert per MFMA
 *                         tile: 0 (the library's choice: 64 while experts
 *                         average fewer than 24 pairs, 128 below 64, else
 *                         192), 64, 128 or 192 (every height computes the
 *                         same bits: it only changes how an expert's pairs
 *                         are split into work items);
 *   gemv_units_per_wg     64-row slabs one GEMV workgroup streams back to
 *                         back: 0 (the library's choice), 1, 2 or 4;
 *   gemv_lanes_per_row    lanes sharing one GEMV weight row: 0 (the
 *                         library's choice), 8 or 32 (32 applies to passes
 *                         of at most 2 token rows);
 *   w2_fused_max_m        self-routed calls with M at or below this run w2
 *                         and the top-k sum as one kernel (an expert shared
 *                         by several tokens is then read once per token):
 *                         0 (the library's choice: 4) or a token count.
 *   mfma_row_tiles        256-row weight tiles of one token tile that one MFMA
 *                         workgroup runs in turn, its loads streaming on across
 *                         them: 0 (the library's choice per GEMM: by the
 *                         work per tile for 128- and 192-slot tiles, 256 rows
 *                         for w13 and 512 for w2 with 64-slot tiles) or 1..16
 *                         for both (results are bit-identical for every
 *                         value).
 * Every choice computes the same function; the
 * GEMV and MFMA kernels differ only in rounding (within the tolerance of
 * fused_experts).  A NULL tuning selects w4a16_moe_default_tuning's values.
 */
typedef struct w4a16_moe_tuning {
  int32_t gemv_only_max_m;
  int32_t gemv_max_tokens;
  int32_t gemv_tokens_per_pass;
  int32_t mfma_tile_m;
  int32_t gemv_units_per_wg;
  int32_t gemv_lanes_per_row;
  int32_t w2_fused_max_m;
  int32_t mfma_row_tiles;
} w4a16_moe_tuning;

/* The built-in tuning for a shape (what NULL selects).  No counterpart in the
 * reference, whose defaults live in kernels/w4a16_moe.py:686-689. */
int w4a16_moe_default_tuning(int64_t M, int64_t topk, int64_t num_experts,
                             int64_t N, int64_t K, int64_t group_size,
                             w4a16_moe_tuning* tuning);

/* w4a16_moe_workspace_size for calls made with `tuning`. */
int w4a16_moe_workspace_size_ex(int64_t M, int64_t topk, int64_t num_experts,
                                int64_t N, int64_t K, int64_t group_size,
                                const w4a16_moe_tuning* tuning, size_t* bytes);

/* w4a16_moe_workspace_layout for calls made with `tuning` (a tuned MFMA tile
 * height or GEMV split changes the sizes of the work lists). */
int w4a16_moe_workspace_layout_ex(int64_t M, int64_t topk, int64_t num_experts,
                                  int64_t N, int64_t K, int64_t group_size,
                                  const w4a16_moe_tuning* tuning,
                                  size_t offsets[W4A16_WS_NFIELDS]);

/* Kernel launches each stage of a call with this shape and tuning enqueues:
 * launches[4] = {expert sort, w13, w2, combine}; 0 = the stage launches
 * nothing (e.g. no sort for self-routed decode, no combine when w2 and the
 * top-k sum run as one kernel).  Assumes 16-byte aligned scale pointers.
 * Measurement helper; no counterpart in the reference. */
int w4a16_moe_stage_launches(int64_t M, int64_t topk, int64_t num_experts,
                             int64_t N, int64_t K, int64_t group_size,
                             const w4a16_moe_tuning* tuning, int32_t launches[4]);

/* w4a16_moe_fused_experts with explicit dispatch choices: the block_m /
 * block_n / block_k arguments of fused_experts_w4a16,
 * kernels/w4a16_moe.py:686-689.  The workspace must hold
 * w4a16_moe_workspace_size_ex(..., tuning) bytes. */
int w4a16_moe_fused_experts_ex(const void* hidden, int64_t ld_hidden,
                               const void* w13_packed, const void* w2_packed,
                               const void* w13_scale, const void* w2_scale,
                               const float* topk_weights, const int32_t* topk_ids,
                               int64_t M, int64_t topk, int64_t num_experts,
                               int64_t N, int64_t K, int64_t group_size,
                               void* out, int64_t ld_out, void* workspace,
                               size_t workspace_bytes, void* stream,
                               const w4a16_moe_tuning* tuning);

/*
 * w4a16_moe_fused_experts_ex with no workspace argument: the call's scratch
 * is a static device array of W4A16_NOALLOC_SCRATCH_BYTES (64 MiB) inside
 * the library, one per device, held until the process ends.  No counterpart
 * in the reference: this entry point is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts
 * that forbid allocation); it calls no hipMalloc/hipFree or allocating
 * library routine.  The caller still passes the inputs and `out`.
 *   - Calls whose workspace (w4a16_moe_workspace_size_ex) exceeds the scratch
 *     return W4A16_ERR_SCRATCH_TOO_SMALL before any GPU work (at E=256,
 *     top-10, K=3072, N=1024 the limit is M <= 818).
 *   - `stream`'s device must be the current device (W4A16_ERR_WRONG_DEVICE
 *     otherwise, before any GPU work).  The first call on a device resolves
 *     the scratch's address there (outside graph capture).
 *   - Every call on one device shares that device's scratch and keeps the
 *     last call's contents: calls that overlap on one device (two streams,
 *     two host threads, two graphs replayed concurrently) race.
 */
int w4a16_moe_fused_experts_noalloc(const void* hidden, int64_t ld_hidden,
                                    const void* w13_packed, const void* w2_packed,
                                    const void* w13_scale, const void* w2_scale,
                                    const float* topk_weights, const int32_t* topk_ids,
                                    int64_t M, int64_t topk, int64_t num_experts,
                                    int64_t N, int64_t K, int64_t group_size,
                                    void* out, int64_t ld_out, void* stream,
                                    const w4a16_moe_tuning* tuning);

/* w4a16_moe_run_stage with explicit dispatch choices (measurement helper). */
int w4a16_moe_run_stage_ex(int stage, const void* hidden, int64_t ld_hidden,
                           const void* w13_packed, const void* w2_packed,
                           const void* w13_scale, const void* w2_scale,
                           const float* topk_weights, const int32_t* topk_ids,
                           int64_t M, int64_t topk, int64_t num_experts,
                           int64_t N, int64_t K, int64_t group_size, void* out,
                           int64_t ld_out, void* workspace,
                           size_t workspace_bytes, void* stream,
                           const w4a16_moe_tuning* tuning);

/* ---- router step (the MoE layer's left neighbour) ----------------------- */
#define W4A16_LOGITS_F32      0
#define W4A16_LOGITS_BF16     1
#define W4A16_ROUTER_MAX_TOPK 64

/*
 * Top-k expert selection and weights from router logits [M, E] (row stride
 * ld_logits elements, fp32 or bf16).
 * Replaces the routing of make_routing, bench/bench_moe.py:225-230:
 *   vals, ids = torch.topk(logits, k);  weights = torch.softmax(vals)
 * topk_ids[M, topk] int32 holds each row's experts by descending logit, equal
 * logits in ascending expert index (torch.topk leaves that order
 * unspecified); NaN ranks above +inf and -0.0 equals +0.0, as in torch.topk.
 * renormalize = 1: topk_weights[M, topk] fp32 = softmax over the k selected
 * logits (the reference).  renormalize = 0: the softmax over all E logits,
 * read at the selected experts.
 * Requirements: 1 <= E <= 1024, 1 <= topk <= min(64, E), ld_logits >= E.
 * One kernel launch on `stream`; M = 0 launches nothing.
 */
int w4a16_moe_router_topk_softmax(const void* logits, int logits_dtype,
                                  int64_t ld_logits, int64_t M,
                                  int64_t num_experts, int64_t topk,
                                  int renormalize, float* topk_weights,
                                  int32_t* topk_ids, void* stream);

/* Human-readable text of a status code (static storage). */
const char* w4a16_moe_strerror(int status);

/* ABI version of this header: 1. */
int w4a16_moe_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_MOE_H */
