/*
 * dsa_indexer.h - C ABI of the DSA index scorer in libdsa_mla.so: the score
 * stage in front of dsa_topk_indices, which together produce the top-k
 * `indices` that dsa_mla_decode consumes.
 *
 * The reference has no indexer: its kernels take lists the caller built
 * ("top-k semantics should already be reflected in kv_indices",
 * opus_attn/dsa_v4/README.md:185-186).  This is the DeepSeek-V3.2 lightning
 * indexer's score, in bf16 with fp32 accumulation:
 *
 *   score[b][t][j] = sum_h  weights[b][t][h] * max(0, q[b][t][h] . k[j])
 *
 * for query token t of sequence b, index head h < H_I, and position j of the
 * sequence, with 128-value index vectors (q: one per token and index head; k:
 * one per cached position, in its own paged cache beside the latent cache).
 * Any scaling (the softmax scale, 1/sqrt(H_I)) is folded into the weights.
 *
 * Positions and pages follow dsa_mla_decode's top-k form: position j of
 * sequence b is scored iff j < len(b, t), len(b, t) = seq_lens[b] -
 * (causal ? s_q - 1 - t : 0), and j < n_cols; its k row is
 *   block_table[b * block_table_stride + j / block_size] * block_size
 *       + j % block_size                      (block_table != NULL)
 *   b * k_batch_stride + j                    (block_table == NULL).
 * A position whose k row lies outside [0, k_total_rows) scores -inf (never
 * worth a top-k slot: dsa_mla_decode skips that row), and is never read.
 *
 * The scores land in score[(b * s_q + t) * score_stride + j] for the scored
 * positions; the others are not written.  dsa_topk_indices then selects over
 * the same rows with lengths len(b, t).
 */
#ifndef DSA_INDEXER_H_
#define DSA_INDEXER_H_

#include <stddef.h>
#include <stdint.h>

#include "dsa_mla.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_INDEXER_D 128        /* index vector length */

typedef struct {
    const void* q;               /* bf16 [B, s_q, H_I, 128], strides in elements (last dim dense) */
    int64_t q_stride_b, q_stride_t, q_stride_h;
    const float* weights;        /* fp32 [B, s_q, H_I] dense */
    const void* k_cache;         /* bf16 [k_total_rows, 128], rows k_stride_row elements apart (0 = 128) */
    int64_t k_total_rows;
    int64_t k_stride_row;
    const int32_t* block_table;  /* as dsa_mla_decode_args (may be NULL) */
    int64_t block_table_stride;
    int32_t block_size;
    int64_t k_batch_stride;
    const int32_t* seq_lens;     /* int32 [B] */
    float* scores;               /* fp32, row (b * s_q + t) at scores + row * score_stride */
    int64_t score_stride;
    int32_t B, s_q, H_I;         /* H_I: 32, 64 or 128 (other counts: DSA_ERR_UNSUPPORTED) */
    int32_t n_cols;              /* positions scored per row: j < min(len, n_cols) */
    int32_t causal;
} dsa_indexer_args;

/*
 * Score every (query token, position) pair on `stream`.  Replaces nothing in
 * the reference (see above).  Returns 0 or a DSA_ERR_* code; validates all
 * arguments before any launch.
 */
int dsa_indexer_scores(const dsa_indexer_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_INDEXER_H_ */
