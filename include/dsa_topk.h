/*
 * DSA top-k index selection on gfx950: the step that produces the `indices`
 * rows the sparse-MLA decode and prefill entries of dsa_mla.h consume.
 *
 * The reference has no counterpart: its attention kernels take kv_indices
 * that the caller has already built ("top-k semantics should already be
 * reflected in kv_indices", opus_attn/dsa_v4/README.md:185; the caller owns
 * the page table, opus_attn/dsa_v32/README.md:99).  This entry is the
 * producer side of that boundary.
 */
#ifndef DSA_TOPK_H_
#define DSA_TOPK_H_

#include <stdint.h>

#include "dsa_mla.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Largest row length (positions) dsa_topk_indices accepts. */
#define DSA_TOPK_MAX_N 0x7ffffff0

/*
 * For each of n_tokens query tokens t, select the topk positions of
 * scores[t, 0:n_t] with the highest scores and write them to
 * indices[t, 0:topk] in ascending position order; when n_t < topk the
 * remaining entries are -1.
 *   scores   fp32 [n_tokens, score_stride] device memory, 16-byte aligned,
 *            score_stride a multiple of 4 and >= n_max.  Row t is read in
 *            16-byte pieces up to n_t rounded up to a multiple of 4.
 *   lengths  int32 [n_tokens] device memory: n_t = clamp(lengths[t], 0, n_max);
 *            NULL means n_t = n_max for every token.  For causal decode with
 *            MTP, token j of a batch with sequence length L passes
 *            L - s_q + j + 1.
 *   indices  int32 [n_tokens, idx_stride], idx_stride >= topk.
 * Order: scores compare as IEEE values, with every NaN above +inf and -0 equal
 * to +0.  Among equal scores at the threshold, lower positions are taken
 * first, so the result is deterministic.  Returns DSA_OK or a DSA_ERR_* code
 * (checked before any launch); topk == 0 or n_tokens == 0 launches nothing.
 */
int dsa_topk_indices(const float* scores, int64_t score_stride, const int32_t* lengths, int32_t n_tokens,
                     int32_t n_max, int32_t topk, int32_t* indices, int64_t idx_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_TOPK_H_ */
