/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, never part of the product path.
 *
 * Plain-C restatement of moe_align_block_size (reference:
 * kernels/w4a16_moe.py:187-290) written as a textbook stable counting sort,
 * i.e. a different formulation from the reference's torch op sequence
 * (histogram :243-249, padded cumsum :251-261, stable sort + amin rank
 * :263-278, searchsorted :280-288).  The Python oracle restates that op
 * sequence literally; the tests require both to agree bit for bit.
 *
 * Contract (identical to the product's): ids outside [0, E) are skipped and
 * counted in *dropped; the reference would index out of bounds on them.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int oracle_align_block_size(const int32_t* ids, int64_t n_tok, int64_t num_experts,
                            int64_t block, int32_t* sorted, int64_t em,
                            int32_t* expert_ids, int64_t n_blocks,
                            int32_t* num_post, int32_t* offsets, int32_t* dropped) {
  if (num_experts < 1 || block < 1 || n_tok < 0) return 1;
  int64_t* cnt = (int64_t*)calloc((size_t)num_experts, sizeof(int64_t));
  int64_t* off = (int64_t*)calloc((size_t)num_experts + 1, sizeof(int64_t));
  int64_t* fill = (int64_t*)calloc((size_t)num_experts, sizeof(int64_t));
  if (!cnt || !off || !fill) {
    free(cnt); free(off); free(fill);
    return 2;
  }
  int64_t drop = 0;
  for (int64_t f = 0; f < n_tok; ++f) {
    const int32_t e = ids[f];
    if (e >= 0 && e < num_experts) ++cnt[e]; else ++drop;
  }
  /* padded per-expert extent, exclusive prefix */
  for (int64_t e = 0; e < num_experts; ++e)
    off[e + 1] = off[e] + (cnt[e] + block - 1) / block * block;
  if (off[num_experts] > em) {
    free(cnt); free(off); free(fill);
    return 3;
  }
  for (int64_t p = 0; p < em; ++p) sorted[p] = (int32_t)n_tok;
  /* stable scatter: ascending flat index within each expert */
  for (int64_t e = 0; e < num_experts; ++e) fill[e] = off[e];
  for (int64_t f = 0; f < n_tok; ++f) {
    const int32_t e = ids[f];
    if (e >= 0 && e < num_experts) sorted[fill[e]++] = (int32_t)f;
  }
  /* block -> expert: expert e owns blocks [off[e]/B, off[e+1]/B) */
  for (int64_t b = 0; b < n_blocks; ++b) expert_ids[b] = -1;
  for (int64_t e = 0; e < num_experts; ++e)
    for (int64_t p = off[e]; p < off[e + 1]; p += block) expert_ids[p / block] = (int32_t)e;
  *num_post = (int32_t)off[num_experts];
  if (offsets)
    for (int64_t e = 0; e <= num_experts; ++e) offsets[e] = (int32_t)off[e];
  if (dropped) *dropped = (int32_t)drop;
  free(cnt); free(off); free(fill);
  return 0;
}
