/*
 * dsa_oracle.c - CPU oracle for the DSA sparse-MLA decode / prefill path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP library is
 * compared against; it is loaded only by tests/, by __graft_entry__.smoke()
 * and by bench.py's cpu_baseline leg, never by the product library.
 *
 * It restates the reference's CPU path in plain C (the reference's own
 * functions live inside host.cc, which needs the un-vendored OPUS headers, so
 * they cannot be compiled here):
 *   - e4m3 codec .................. opus_attn/dsa_v32/common/defs.h:11-52
 *   - attention core .............. opus_attn/dsa_v32/common/host.cc:431-457
 *                                   (sm_scale is a parameter instead of the
 *                                   hard-coded 1/sqrt(576) at :437)
 *   - per-token decode reference .. opus_attn/dsa_v32/common/host.cc:459-548,
 *                                   with the gather-once-per-token structure of
 *                                   opus_attn/dsa_v41/common/mla_v41_host.cc:458-517
 *   - per-query prefill reference . opus_attn/dsa_v4/common/mla_v4_host.cc:482-532
 *                                   (no sink: sink = -inf reduces :469,:472 to
 *                                   the decode core)
 *   - V4 prefill (prefix + extend
 *     pools, attention sink, D=512) opus_attn/dsa_v4/common/mla_v4_host.cc:455-532
 *   - MXFP8 split-stream decode ... opus_attn/dsa_v32/common/host.cc:418-429 (dequant),
 *                                   :459-506 (CSR rows, count-based MTP causality)
 *   - V4 fp8 prefill .............. opus_attn/dsa_v4/common/mla_v4_host.cc:443-453 (dequant),
 *                                   :535-588 (prefix + extend rows, sink)
 *   - split combine ............... opus_attn/dsa_v32/common/mla_reduce.hpp:6-156
 *   - threading ................... opus_attn/dsa_v32/common/parallel.h:11-57
 * generalised to the top-k index form (-1 padding, seq_len and causal bounds,
 * paged block table) and the 656-byte fp8 row.
 *
 * Pinning (tests/test_oracle_*.py): the e4m3 codec exhaustively against the
 * OCP E4M3FN closed form and brute-force nearest rounding; bf16 rounding
 * against torch; the attention core against fp64 numpy brute force on small
 * shapes and against closed forms (single index, identical rows, q = 0, all
 * invalid); index handling by exact equality with filtered lists; the combine
 * by split-vs-unsplit identity.
 */
#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "../include/dsa_mla.h"

#define D_QK DSA_MLA_D_QK
#define D_NOPE DSA_MLA_D_NOPE
#define D_ROPE DSA_MLA_D_ROPE
#define D_VO DSA_MLA_D_VO

/* ---------------------------------------------------------------- codecs */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fp32 -> bf16 bits, round to nearest even; NaN -> quiet NaN. */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/*
 * fp32 -> OCP e4m3fn code, round to nearest even, saturating to +-448,
 * Inf/NaN -> 0x7F | sign.  Same decision points as defs.h:11-38: magnitude
 * >= 448 saturates, normal range keeps 3 mantissa bits, values below 2^-6
 * go to the subnormal grid of step 2^-9, below 2^-17 flush to signed zero.
 */
uint8_t oracle_fp8_e4m3_encode(float f) {
    const uint32_t bits = f2u(f);
    const uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
    const uint32_t mag = bits & 0x7FFFFFFFu;
    if (mag >= 0x7F800000u) return (uint8_t)(sign | 0x7Fu);
    if (mag >= 0x43E00000u) return (uint8_t)(sign | 0x7Eu); /* >= 448 */
    const int e = (int)(mag >> 23) - 127;
    uint32_t code, rest, half;
    if (e >= -6) {
        const uint32_t m = mag & 0x7FFFFFu;
        code = ((uint32_t)(e + 7) << 3) | (m >> 20);
        rest = m & 0xFFFFFu;
        half = 0x80000u;
    } else {
        const int sh = -6 - e; /* extra right shift into the subnormal grid */
        if (sh > 11) return sign;
        const uint32_t m = (mag & 0x7FFFFFu) | 0x800000u;
        const uint32_t w = 20u + (uint32_t)sh;
        code = m >> w;
        rest = m & ((1u << w) - 1u);
        half = 1u << (w - 1u);
    }
    if (rest > half || (rest == half && (code & 1u))) code++;
    return (uint8_t)(sign | code);
}

/* OCP e4m3fn code -> fp32 (defs.h:40-52): NaN for S.1111.111. */
float oracle_fp8_e4m3_decode(uint8_t c) {
    const uint32_t s = (uint32_t)(c & 0x80u) << 24;
    const uint32_t e = (c >> 3) & 0xFu;
    const uint32_t m = c & 7u;
    if (e == 15u && m == 7u) return u2f(s | 0x7FC00000u);
    if (e == 0u) {
        const float v = (float)m * (1.0f / 512.0f);
        return (c & 0x80u) ? -v : v;
    }
    return u2f(s | ((e + 120u) << 23) | (m << 20));
}

void oracle_fp8_encode_n(const float* x, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_e4m3_encode(x[i]);
}
void oracle_fp8_decode_n(const uint8_t* c, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_e4m3_decode(c[i]);
}
void oracle_bf16_round_n(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(x[i]);
}

/*
 * 656-byte row writer: src is 576 fp32 values (the bf16 latent widened).
 * scale_g = amax_g / 448 (IEEE division), code = e4m3(x / scale_g); an
 * all-zero group stores scale 0 and zero codes.  RoPE is rounded to bf16.
 */
void oracle_quantize_row_656(const float* src, uint8_t* dst) {
    for (int g = 0; g < 4; ++g) {
        float amax = 0.0f;
        for (int i = 0; i < 128; ++i) {
            const float a = fabsf(src[128 * g + i]);
            if (a > amax) amax = a;
        }
        const float scale = amax / 448.0f;
        memcpy(dst + 512 + 4 * g, &scale, 4);
        for (int i = 0; i < 128; ++i)
            dst[128 * g + i] = (scale > 0.0f) ? oracle_fp8_e4m3_encode(src[128 * g + i] / scale) : 0;
    }
    for (int i = 0; i < D_ROPE; ++i) {
        const uint16_t h = oracle_f32_to_bf16(src[D_NOPE + i]);
        memcpy(dst + 528 + 2 * i, &h, 2);
    }
}

void oracle_quantize_rows_656(const float* src, int64_t n, uint8_t* dst) {
    for (int64_t r = 0; r < n; ++r) oracle_quantize_row_656(src + r * D_QK, dst + r * 656);
}

/* 656-byte row -> 576 fp32 (the fp8 analogue of host.cc:418-429). */
void oracle_dequant_row_656(const uint8_t* row, float* out) {
    float scale[4];
    memcpy(scale, row + 512, 16);
    for (int d = 0; d < D_NOPE; ++d) out[d] = oracle_fp8_e4m3_decode(row[d]) * scale[d / 128];
    for (int j = 0; j < D_ROPE; ++j) {
        uint16_t h;
        memcpy(&h, row + 528 + 2 * j, 2);
        out[D_NOPE + j] = oracle_bf16_to_f32(h);
    }
}

void oracle_dequant_rows_656(const uint8_t* rows, int64_t n, float* out) {
    for (int64_t r = 0; r < n; ++r) oracle_dequant_row_656(rows + r * 656, out + r * D_QK);
}

/* Bytes between cache rows: stride in elements of the row format (bf16
 * elements, or bytes for 656-B rows), 0 = dense rows (defs.h:129). */
static int64_t row_stride_bytes(int fmt, int64_t stride) {
    if (fmt == DSA_KV_BF16) return stride ? 2 * stride : DSA_MLA_BF16_ROW_BYTES;
    return stride ? stride : DSA_MLA_FP8_ROW_BYTES;
}

static void load_row(const uint8_t* cache, int fmt, int64_t row_bytes, int64_t row, float* out) {
    if (fmt == DSA_KV_BF16) {
        const uint16_t* p = (const uint16_t*)(cache + row * row_bytes);
        for (int d = 0; d < D_QK; ++d) out[d] = oracle_bf16_to_f32(p[d]);
    } else {
        oracle_dequant_row_656(cache + row * row_bytes, out);
    }
}

/* ------------------------------------------------------ attention core */

/*
 * scores[p] = (q . row_p) * scale over n rows of width D (row stride D), each
 * dot product summed in dim order, one fp32 multiply then one add per dim, as
 * host.cc:437-438 and mla_v4_host.cc:463-466 write it.  Four rows at a time:
 * their four sums are independent, so they overlap, and every row's sum sees
 * exactly the operations of the one-row loop.
 */
static void dot_rows(const float* q, const float* kv, int n, int D, float scale, float* scores) {
    int p = 0;
    for (; p + 4 <= n; p += 4) {
        const float* k0 = kv + (size_t)p * D;
        const float* k1 = k0 + D;
        const float* k2 = k1 + D;
        const float* k3 = k2 + D;
        float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
        for (int d = 0; d < D; ++d) {
            const float x = q[d];
            d0 += x * k0[d];
            d1 += x * k1[d];
            d2 += x * k2[d];
            d3 += x * k3[d];
        }
        scores[p] = d0 * scale;
        scores[p + 1] = d1 * scale;
        scores[p + 2] = d2 * scale;
        scores[p + 3] = d3 * scale;
    }
    for (; p < n; ++p) {
        const float* k = kv + (size_t)p * D;
        float dot = 0.0f;
        for (int d = 0; d < D; ++d) dot += q[d] * k[d];
        scores[p] = dot * scale;
    }
}

/*
 * acc[d] = sum_p w[p] * row_p[d] for d < D (rows `stride` floats apart), each
 * sum taken over the rows in list order from 0.0f, as host.cc:452-456 and
 * mla_v4_host.cc:473-477 write it.  Rows outer, dims inner: the rows are read
 * once, in order, and every output sees exactly the operations of the
 * dims-outer loop.
 */
static void weighted_rows(const float* w, const float* kv, int n, int stride, int D, float* acc) {
    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
    for (int p = 0; p < n; ++p) {
        const float s = w[p];
        const float* r = kv + (size_t)p * stride;
        for (int d = 0; d < D; ++d) acc[d] += s * r[d];
    }
}

/*
 * One (token, head): host.cc:431-457 with sm_scale as a parameter.
 * Writes either the final row (o_bf16 != NULL: bf16 O and LSE, O = 0 and
 * LSE = +inf when n == 0, host.cc:486-489) or a split partial (o_f32: fp32 O
 * normalised by the split's own sum and its natural-log LSE, -FLT_MAX when
 * empty, as the partial path of the decode kernel stores for mla_reduce).
 */
static void attention_core(const float* q, const float* kv, int n, float sm_scale, float* scores,
                           uint16_t* o_bf16, float* o_f32, float* lse) {
    if (n <= 0) {
        for (int d = 0; d < D_VO; ++d) {
            if (o_bf16) o_bf16[d] = 0;
            if (o_f32) o_f32[d] = 0.0f;
        }
        if (lse) *lse = o_bf16 ? INFINITY : -FLT_MAX;
        return;
    }
    dot_rows(q, kv, n, D_QK, sm_scale, scores);
    float mx = scores[0];
    for (int p = 1; p < n; ++p) if (scores[p] > mx) mx = scores[p];
    float sum = 0.0f;
    for (int p = 0; p < n; ++p) { scores[p] = expf(scores[p] - mx); sum += scores[p]; }
    if (lse) *lse = logf(sum) + mx;
    for (int p = 0; p < n; ++p) scores[p] = oracle_bf16_to_f32(oracle_f32_to_bf16(scores[p] / sum));
    float acc[D_VO];
    weighted_rows(scores, kv, n, D_QK, D_VO, acc);
    for (int d = 0; d < D_VO; ++d) {
        if (o_bf16) o_bf16[d] = oracle_f32_to_bf16(acc[d]);
        if (o_f32) o_f32[d] = acc[d];
    }
}

/* ------------------------------------------------------------ threading */

typedef void (*task_fn)(void* ctx, int64_t i, float* scratch);

typedef struct {
    task_fn fn;
    void* ctx;
    int64_t n;
    int64_t next;
    pthread_mutex_t mu;
    size_t scratch_floats;
} pool_t;

static void* pool_worker(void* arg) {
    pool_t* p = (pool_t*)arg;
    float* scratch = (float*)malloc(p->scratch_floats * sizeof(float));
    if (!scratch) return NULL;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        const int64_t i = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (i >= p->n) break;
        p->fn(p->ctx, i, scratch);
    }
    free(scratch);
    return NULL;
}

/* parallel.h:11-18: explicit count, else DSA_ORACLE_NUM_THREADS, else all cores. */
int oracle_num_threads(int requested) {
    if (requested > 0) return requested;
    const char* env = getenv("DSA_ORACLE_NUM_THREADS");
    if (env && atoi(env) > 0) return atoi(env);
    const long hw = sysconf(_SC_NPROCESSORS_ONLN);
    return hw > 0 ? (int)hw : 1;
}

static int run_pool(task_fn fn, void* ctx, int64_t n, size_t scratch_floats, int nthreads) {
    pool_t p;
    p.fn = fn; p.ctx = ctx; p.n = n; p.next = 0; p.scratch_floats = scratch_floats;
    pthread_mutex_init(&p.mu, NULL);
    int nt = oracle_num_threads(nthreads);
    if (nt > n) nt = (int)(n > 0 ? n : 1);
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nt);
    if (!th) return -1;
    for (int t = 1; t < nt; ++t) pthread_create(&th[t], NULL, pool_worker, &p);
    pool_worker(&p);
    for (int t = 1; t < nt; ++t) pthread_join(th[t], NULL);
    free(th);
    pthread_mutex_destroy(&p.mu);
    return 0;
}

/* --------------------------------------------------------------- decode */

typedef struct {
    const dsa_mla_decode_args* a;
    int32_t k_begin, k_end;      /* top-k sub-range [k_begin, k_end) */
    float* part_o;               /* fp32 [B*s_q, H, 512] or NULL (final mode) */
    float* part_lse;             /* fp32 [B*s_q, H] */
} decode_ctx;

/* Physical row of logical position j of (b, t) or -1 if invalid. */
static int64_t resolve(const dsa_mla_decode_args* a, int b, int t, int32_t j) {
    const int32_t L = a->seq_lens[b];
    if (j < 0 || j >= L) return -1;
    if (a->causal && j > L - a->s_q + t) return -1;
    int64_t row;
    if (a->block_table) {
        const int32_t blk = a->block_table[(int64_t)b * a->block_table_stride + j / a->block_size];
        row = (int64_t)blk * a->block_size + j % a->block_size;
    } else {
        row = (int64_t)b * a->kv_batch_stride + j;
    }
    if (row < 0 || row >= a->kv_total_rows) return -1;
    return row;
}

static void decode_task(void* vctx, int64_t i, float* scratch) {
    const decode_ctx* c = (const decode_ctx*)vctx;
    const dsa_mla_decode_args* a = c->a;
    const int b = (int)(i / a->s_q), t = (int)(i % a->s_q);
    const int32_t* idx = a->indices + b * a->idx_stride_b + t * a->idx_stride_t;
    float* q = scratch;
    float* scores = q + D_QK;
    float* kv = scores + a->topk;
    /* gather every valid row once per token (mla_v41_host.cc:458-517) */
    int n = 0;
    for (int k = c->k_begin; k < c->k_end; ++k) {
        const int64_t row = resolve(a, b, t, idx[k]);
        if (row < 0) continue;
        load_row((const uint8_t*)a->kv_cache, a->kv_format, row_stride_bytes(a->kv_format, a->kv_stride_row), row,
                 kv + (size_t)n * D_QK);
        ++n;
    }
    const uint16_t* qb = (const uint16_t*)a->q;
    for (int h = 0; h < a->H; ++h) {
        const uint16_t* qs = qb + b * a->q_stride_b + t * a->q_stride_t + h * a->q_stride_h;
        for (int d = 0; d < D_QK; ++d) q[d] = oracle_bf16_to_f32(qs[d]);
        if (c->part_o) {
            const int64_t r = i * a->H + h;
            attention_core(q, kv, n, a->sm_scale, scores, NULL, c->part_o + r * D_VO,
                           c->part_lse + r);
        } else {
            uint16_t* o = (uint16_t*)a->out + b * a->o_stride_b + t * a->o_stride_t + h * a->o_stride_h;
            attention_core(q, kv, n, a->sm_scale, scores, o, NULL,
                           a->lse ? a->lse + i * a->H + h : NULL);
        }
    }
}

/* Final decode over the whole top-k list: bf16 O and fp32 LSE (host pointers). */
int oracle_mla_decode(const dsa_mla_decode_args* a, int nthreads) {
    decode_ctx c = {a, 0, a->topk, NULL, NULL};
    const size_t scratch = (size_t)D_QK + a->topk + (size_t)a->topk * D_QK;
    return run_pool(decode_task, &c, (int64_t)a->B * a->s_q, scratch, nthreads);
}

/* Split partial over top-k range [k_begin, k_end): fp32 O and LSE per (token, head). */
int oracle_mla_decode_partial(const dsa_mla_decode_args* a, int32_t k_begin, int32_t k_end,
                              float* part_o, float* part_lse, int nthreads) {
    decode_ctx c = {a, k_begin, k_end, part_o, part_lse};
    const size_t scratch = (size_t)D_QK + a->topk + (size_t)a->topk * D_QK;
    return run_pool(decode_task, &c, (int64_t)a->B * a->s_q, scratch, nthreads);
}

/* -------------------------------------------------------------- combine */

/*
 * mla_reduce.hpp:6-156: m = max lse_i, w_i = exp(lse_i - m) (0 for an empty
 * split), O = sum w_i O_i / sum w_i, LSE = m + ln(sum w_i), +inf and O = 0
 * when every split is empty.  Evaluated in double for a tight reference.
 */
void oracle_mla_combine(const float* part_o, const float* part_lse, int32_t ns, int64_t rows,
                        int32_t H, uint16_t* out, float* lse) {
    for (int64_t r = 0; r < rows * H; ++r) {
        double m = -DBL_MAX;
        for (int s = 0; s < ns; ++s) {
            const float l = part_lse[(int64_t)s * rows * H + r];
            if (l > -FLT_MAX && l > m) m = l;
        }
        double den = 0.0;
        double acc[D_VO];
        for (int d = 0; d < D_VO; ++d) acc[d] = 0.0;
        for (int s = 0; s < ns; ++s) {
            const float l = part_lse[(int64_t)s * rows * H + r];
            if (!(l > -FLT_MAX)) continue;
            const double w = exp((double)l - m);
            den += w;
            const float* o = part_o + ((int64_t)s * rows * H + r) * D_VO;
            for (int d = 0; d < D_VO; ++d) acc[d] += w * o[d];
        }
        for (int d = 0; d < D_VO; ++d)
            out[r * D_VO + d] = oracle_f32_to_bf16(den > 0.0 ? (float)(acc[d] / den) : 0.0f);
        if (lse) lse[r] = den > 0.0 ? (float)(m + log(den)) : INFINITY;
    }
}

/* -------------------------------------------------------------- prefill */

typedef struct {
    const dsa_mla_prefill_args* a;
} prefill_ctx;

static void prefill_task(void* vctx, int64_t i, float* scratch) {
    const dsa_mla_prefill_args* a = ((const prefill_ctx*)vctx)->a;
    const int32_t* idx = a->indices + i * a->idx_stride_n;
    float* q = scratch;
    float* scores = q + D_QK;
    float* kv = scores + a->topk;
    int n = 0;
    for (int k = 0; k < a->topk; ++k) {
        const int32_t j = idx[k];
        if (j < 0 || j >= a->kv_rows) continue;
        if (a->causal && (int64_t)j > i + a->causal_offset) continue;
        load_row((const uint8_t*)a->kv, a->kv_format, row_stride_bytes(a->kv_format, a->kv_stride_row), j,
                 kv + (size_t)n * D_QK);
        ++n;
    }
    const uint16_t* qb = (const uint16_t*)a->q;
    for (int h = 0; h < a->H; ++h) {
        const uint16_t* qs = qb + i * a->q_stride_n + h * a->q_stride_h;
        for (int d = 0; d < D_QK; ++d) q[d] = oracle_bf16_to_f32(qs[d]);
        uint16_t* o = (uint16_t*)a->out + i * a->o_stride_n + h * a->o_stride_h;
        attention_core(q, kv, n, a->sm_scale, scores, o, NULL, a->lse ? a->lse + i * a->H + h : NULL);
    }
}

/* ------------------------------------------------------- V4 prefill */

/*
 * mla_v4_attention_compute (opus_attn/dsa_v4/common/mla_v4_host.cc:455-480)
 * with softmax_scale as a parameter (:461 hard-codes 1/sqrt(D)): scores in
 * fp32, max over the scores and the sink, denominator sum exp(s - max) +
 * exp(sink - max), P rounded to bf16 after normalisation, O = P . rows
 * (V = the whole 512-value row) cast to bf16.  LSE = max + ln(denominator),
 * an addition of this build; a query with no rows gets O = 0, LSE = +inf.
 */
static void attention_core_v4(const float* q, const float* kv, int n, float scale, float sink,
                              float* scores, uint16_t* o_bf16, float* lse) {
    const int D = DSA_MLA_D_V4;
    if (n <= 0) {
        for (int d = 0; d < D; ++d) o_bf16[d] = 0;
        if (lse) *lse = INFINITY;
        return;
    }
    dot_rows(q, kv, n, D, scale, scores);
    float mx = sink;
    for (int p = 0; p < n; ++p) if (scores[p] > mx) mx = scores[p];
    float sum = 0.0f;
    for (int p = 0; p < n; ++p) { scores[p] = expf(scores[p] - mx); sum += scores[p]; }
    sum += expf(sink - mx);
    if (lse) *lse = logf(sum) + mx;
    for (int p = 0; p < n; ++p) scores[p] = oracle_bf16_to_f32(oracle_f32_to_bf16(scores[p] / sum));
    float acc[DSA_MLA_D_V4];
    weighted_rows(scores, kv, n, D, D, acc);
    for (int d = 0; d < D; ++d) o_bf16[d] = oracle_f32_to_bf16(acc[d]);
}

typedef struct {
    const dsa_mla_prefill_v4_args* a;
} prefill_v4_ctx;

/* mla_v4_attention_ref (mla_v4_host.cc:482-532): prefix rows, then extend rows. */
static void prefill_v4_task(void* vctx, int64_t i, float* scratch) {
    const dsa_mla_prefill_v4_args* a = ((const prefill_v4_ctx*)vctx)->a;
    const int D = DSA_MLA_D_V4;
    float* q = scratch;
    float* scores = q + D;
    float* kv = scores + a->max_rows;
    int n = 0;
    const int32_t pb = a->kv_indptr_prefix[i], pe = a->kv_indptr_prefix[i + 1];
    const int32_t eb = a->kv_indptr_extend[i], ee = a->kv_indptr_extend[i + 1];
    for (int pass = 0; pass < 2; ++pass) {
        const int32_t* ind = pass == 0 ? a->kv_indices_prefix : a->kv_indices_extend;
        const uint16_t* pool = (const uint16_t*)(pass == 0 ? a->unified_kv : a->kv);
        const int32_t rows = pass == 0 ? a->total_pages : a->total_tokens;
        for (int32_t k = pass == 0 ? pb : eb; k < (pass == 0 ? pe : ee) && n < a->max_rows; ++k) {
            const int32_t j = ind[k];
            if (j < 0 || j >= rows) continue;   /* a row outside its pool is skipped */
            const uint16_t* src = pool + (int64_t)j * a->stride_kv_page;
            for (int d = 0; d < D; ++d) kv[(size_t)n * D + d] = oracle_bf16_to_f32(src[d]);
            ++n;
        }
    }
    const uint16_t* qb = (const uint16_t*)a->q;
    for (int h = 0; h < a->H; ++h) {
        const uint16_t* qs = qb + i * a->stride_qo_n + h * a->stride_qo_h;
        for (int d = 0; d < D; ++d) q[d] = oracle_bf16_to_f32(qs[d]);
        uint16_t* o = (uint16_t*)a->out + i * a->stride_qo_n + h * a->stride_qo_h;
        const float sink = a->attn_sink ? a->attn_sink[h] : -INFINITY;
        attention_core_v4(q, kv, n, a->softmax_scale, sink, scores, o, a->lse ? a->lse + i * a->H + h : NULL);
    }
}

int oracle_mla_prefill_v4(const dsa_mla_prefill_v4_args* a, int nthreads) {
    prefill_v4_ctx c = {a};
    const size_t scratch = (size_t)DSA_MLA_D_V4 + a->max_rows + (size_t)a->max_rows * DSA_MLA_D_V4;
    return run_pool(prefill_v4_task, &c, a->N, scratch, nthreads);
}

/* mla_v4_host.cc:482-532 for the V3.2 shape without sink, with LSE. */
int oracle_mla_prefill(const dsa_mla_prefill_args* a, int nthreads) {
    prefill_ctx c = {a};
    const size_t scratch = (size_t)D_QK + a->topk + (size_t)a->topk * D_QK;
    return run_pool(prefill_task, &c, a->N, scratch, nthreads);
}

/* ------------------------------------------------------- MXFP8 decode */

/*
 * dequant_mla_row_fp8 (opus_attn/dsa_v32/common/host.cc:418-429): NoPE dim d
 * = e4m3(code_d) * 2^(scale[d / 32] - 127) (ldexp of the E8M0 byte), RoPE
 * bf16 widened.  Strides in elements of each stream.
 */
void oracle_dequant_row_mxfp8(const uint8_t* nope, const uint8_t* scale, const uint16_t* rope, float* out) {
    for (int d = 0; d < D_NOPE; ++d)
        out[d] = oracle_fp8_e4m3_decode(nope[d]) * ldexpf(1.0f, (int)scale[d / 32] - 127);
    for (int j = 0; j < D_ROPE; ++j) out[D_NOPE + j] = oracle_bf16_to_f32(rope[j]);
}

typedef struct {
    const dsa_mla_decode_mxfp8_args* a;
} mx_ctx;

/*
 * mla_decode_attention_ref_fp8 (host.cc:459-506) for query token row i =
 * b * s_q + t: rows kv_indices[kv_indptr[b] + p] for p < kv_indptr[b+1] -
 * kv_indptr[b] - (s_q - 1 - t) (:481-482), every row and Q dequantised to
 * fp32 (:493-502), then the decode attention core (:431-457) with
 * softmax_scale as a parameter.  A row outside [0, total_tokens) is skipped
 * (the reference reads it unchecked).
 */
static void mx_task(void* vctx, int64_t i, float* scratch) {
    const dsa_mla_decode_mxfp8_args* a = ((const mx_ctx*)vctx)->a;
    const int b = (int)(i / a->s_q), t = (int)(i % a->s_q);
    float* q = scratch;
    float* scores = q + D_QK;
    float* kv = scores + a->max_kv_len;
    const int32_t kb = a->kv_indptr[b];
    const int32_t count = a->kv_indptr[b + 1] - kb - (a->s_q - 1 - t);
    int n = 0;
    for (int32_t p = 0; p < count && p < a->max_kv_len; ++p) {
        const int32_t r = a->kv_indices[kb + p];
        if (r < 0 || r >= a->total_tokens) continue;
        oracle_dequant_row_mxfp8((const uint8_t*)a->kv_nope + (int64_t)r * a->stride_kv_nope_page,
                                 (const uint8_t*)a->kv_scale + (int64_t)r * a->stride_kv_scale_page,
                                 (const uint16_t*)a->kv_rope + (int64_t)r * a->stride_kv_rope_page,
                                 kv + (size_t)n * D_QK);
        ++n;
    }
    for (int h = 0; h < a->H; ++h) {
        oracle_dequant_row_mxfp8((const uint8_t*)a->q_nope + i * a->stride_q_nope_b + h * a->stride_q_nope_h,
                                 (const uint8_t*)a->q_scale + i * a->stride_q_scale_b + h * a->stride_q_scale_h,
                                 (const uint16_t*)a->q_rope + i * a->stride_q_rope_b + h * a->stride_q_rope_h,
                                 q);
        uint16_t* o = (uint16_t*)a->out + i * a->stride_o_b + h * a->stride_o_h;
        attention_core(q, kv, n, a->softmax_scale, scores, o, NULL, a->lse ? a->lse + i * a->H + h : NULL);
    }
}

/* Final MXFP8 decode: bf16 O and fp32 LSE (host pointers); max_kv_len bounds every list. */
int oracle_mla_decode_mxfp8(const dsa_mla_decode_mxfp8_args* a, int nthreads) {
    mx_ctx c = {a};
    const size_t scratch = (size_t)D_QK + a->max_kv_len + (size_t)a->max_kv_len * D_QK;
    return run_pool(mx_task, &c, (int64_t)a->B * a->s_q, scratch, nthreads);
}

/* ------------------------------------------------------- V4 fp8 prefill */

/*
 * decode_dsa_row_fp8 (opus_attn/dsa_v4/common/mla_v4_host.cc:443-453): value
 * d < 448 = e4m3(nope[d]) * 2^(nope[448 + d / 32] - 127) (the scales follow
 * the codes in the 512-byte stream row), values 448..511 the bf16 RoPE.
 */
void oracle_dequant_row_v4fp8(const uint8_t* nope, const uint16_t* rope, float* out) {
    for (int d = 0; d < DSA_MLA_V4_NOPE; ++d)
        out[d] = oracle_fp8_e4m3_decode(nope[d]) * ldexpf(1.0f, (int)nope[DSA_MLA_V4_NOPE + d / 32] - 127);
    for (int j = 0; j < D_ROPE; ++j) out[DSA_MLA_V4_NOPE + j] = oracle_bf16_to_f32(rope[j]);
}

typedef struct {
    const dsa_mla_prefill_v4_fp8_args* a;
} prefill_v4_fp8_ctx;

/*
 * mla_v4_attention_ref_fp8 (mla_v4_host.cc:535-588): Q and every prefix then
 * extend row dequantised to fp32, then mla_v4_attention_compute
 * (:455-480) with softmax_scale as a parameter.  A row outside its pool is
 * skipped (the reference reads it unchecked).
 */
static void prefill_v4_fp8_task(void* vctx, int64_t i, float* scratch) {
    const dsa_mla_prefill_v4_fp8_args* a = ((const prefill_v4_fp8_ctx*)vctx)->a;
    const int D = DSA_MLA_D_V4;
    float* q = scratch;
    float* scores = q + D;
    float* kv = scores + a->max_rows;
    int n = 0;
    const int32_t pb = a->kv_indptr_prefix[i], pe = a->kv_indptr_prefix[i + 1];
    const int32_t eb = a->kv_indptr_extend[i], ee = a->kv_indptr_extend[i + 1];
    for (int pass = 0; pass < 2; ++pass) {
        const int32_t* ind = pass == 0 ? a->kv_indices_prefix : a->kv_indices_extend;
        const uint8_t* nope = (const uint8_t*)(pass == 0 ? a->unified_kv_nope : a->kv_nope);
        const uint16_t* rope = (const uint16_t*)(pass == 0 ? a->unified_kv_rope : a->kv_rope);
        const int32_t rows = pass == 0 ? a->total_pages : a->total_tokens;
        for (int32_t k = pass == 0 ? pb : eb; k < (pass == 0 ? pe : ee) && n < a->max_rows; ++k) {
            const int32_t j = ind[k];
            if (j < 0 || j >= rows) continue;
            oracle_dequant_row_v4fp8(nope + (int64_t)j * a->stride_kv_nope_page,
                                     rope + (int64_t)j * a->stride_kv_rope_page, kv + (size_t)n * D);
            ++n;
        }
    }
    for (int h = 0; h < a->H; ++h) {
        oracle_dequant_row_v4fp8((const uint8_t*)a->q_nope + i * a->stride_q_nope_n + h * a->stride_q_nope_h,
                                 (const uint16_t*)a->q_rope + i * a->stride_q_rope_n + h * a->stride_q_rope_h, q);
        uint16_t* o = (uint16_t*)a->out + i * a->stride_o_n + h * a->stride_o_h;
        const float sink = a->attn_sink ? a->attn_sink[h] : -INFINITY;
        attention_core_v4(q, kv, n, a->softmax_scale, sink, scores, o, a->lse ? a->lse + i * a->H + h : NULL);
    }
}

int oracle_mla_prefill_v4_fp8(const dsa_mla_prefill_v4_fp8_args* a, int nthreads) {
    prefill_v4_fp8_ctx c = {a};
    const size_t scratch = (size_t)DSA_MLA_D_V4 + a->max_rows + (size_t)a->max_rows * DSA_MLA_D_V4;
    return run_pool(prefill_v4_fp8_task, &c, a->N, scratch, nthreads);
}
