/*
 * dsa_mla.h - C ABI of the MI355X (gfx950) DeepSeek sparse-attention (DSA)
 * MLA decode / prefill library, libdsa_mla.so.
 *
 * One latent KV row is 576 values: 512 "NoPE" values (which are also the
 * value vector V) followed by 64 "RoPE" values.  Every query head attends
 * the same gathered rows; the output is 512 wide per head.
 *
 * Row formats in the KV cache (byte layout of one cache row):
 *   DSA_KV_BF16    : 576 x bf16                                  = 1152 B
 *   DSA_KV_FP8_656 : [0,512)   512 x fp8 e4m3fn NoPE codes
 *                    [512,528) 4 x fp32 scales, scale g covers NoPE dims
 *                              [128g, 128g+128) and equals amax_g / 448
 *                    [528,656) 64 x bf16 RoPE                    =  656 B
 *   Dequantised value of NoPE dim d = float(e4m3(code_d)) * scale[d / 128].
 *   Range: the kernels compute these rows in fp16 (K and V values, and Q's
 *   NoPE part).  Any finite q is accepted: a head with |q| >= 2^15 is scaled
 *   by a power of two into fp16's range and its softmax scale by the inverse,
 *   which is exact.  Every scale of an attended row must lie in [0, 128)
 *   (group amax below 57344, so every value stays below fp16's 65504); a
 *   query token that attends a row with a scale of 128 or more, or a negative
 *   or non-finite one, gets NaN O and LSE (a defined signal, never a silently
 *   wrong attention).  Rows the cache writer produces from bf16 inputs with
 *   group amax below 57344 always qualify.
 *
 * Index semantics (top-k form).  indices[b][t][k] is a logical position j in
 * sequence b.  It is valid iff 0 <= j < seq_lens[b] and, when causal != 0,
 * j <= seq_lens[b] - s_q + t.  Invalid entries (-1 padding included)
 * contribute nothing.  The physical cache row of a valid j is
 *   block_table[b * block_table_stride + j / block_size] * block_size
 *       + j % block_size                       (block_table != NULL)
 *   b * kv_batch_stride + j                    (block_table == NULL)
 * and a physical row outside [0, kv_total_rows) is treated as invalid, so a
 * bad block table can never make a kernel read outside the cache.
 * Duplicated positions count once per occurrence.  A (b, t, head) with no
 * valid entry gets O = 0 and LSE = +inf.
 *
 * Heads.  Every entry takes any head count H >= 1 (H <= 0 is
 * DSA_ERR_BAD_SHAPE).  A query token runs in ceil(H / 128) workgroups of 128
 * heads, or, for bf16 and 656-B fp8 rows at H <= 32 or when 128-head
 * workgroups would be too few to occupy the GPU, in ceil(H / 32) workgroups
 * of 32 heads (the
 * summation order of the scores then differs, within the same bounds); the
 * last group computes its heads past H on a copy of head H-1 and stores
 * nothing for them, so outputs, LSEs and partials are written for heads
 * 0..H-1 only.  The kernel choice changes dsa_mla_decode_num_splits and the
 * workspace sizes, which report the split count of the kernel that runs.
 *
 * Numerics.  Scores s = (q . k) * sm_scale in fp32; softmax probabilities are
 * rounded to the P.V product's 16-bit type before it (bf16 for bf16 and MXFP8
 * rows, as the reference does at host.cc:451; fp16 for DSA_KV_FP8_656 rows,
 * whose V is fp16), accumulation is fp32, O is written as bf16 (round to
 * nearest even) and LSE = max + ln(sum exp(s - max)) as fp32 (natural log of
 * the scaled scores).
 *
 * Conventions.  All pointers are device pointers owned by the caller (the
 * workspace included); strides are in elements; `stream` is a hipStream_t
 * (NULL = the null stream).  Every entry point validates its arguments
 * before any launch and returns 0 on success or a negative DSA_ERR_* code;
 * nothing calls exit().  Apart from the device scratch of
 * dsa_mla_decode_noalloc the library holds no mutable global state, so calls
 * on distinct streams with distinct workspaces may run concurrently.
 */
#ifndef DSA_MLA_H_
#define DSA_MLA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_MLA_D_QK 576
#define DSA_MLA_D_NOPE 512
#define DSA_MLA_D_ROPE 64
#define DSA_MLA_D_VO 512
#define DSA_MLA_FP8_ROW_BYTES 656
#define DSA_MLA_BF16_ROW_BYTES 1152
#define DSA_MLA_MAX_SPLITS 64
/* num_splits of the CSR entries: the workspace already holds the work plan
 * of these lists (dsa_mla_csr_plan) */
#define DSA_MLA_SPLITS_PLANNED (-1)
/* longest list an entry takes (top-k, max_kv_len, max_rows): INT32_MAX - 2048 */
#define DSA_MLA_MAX_LIST 2147481599
#define DSA_MLA_D_V4 512       /* V4 prefill head dim: K = V = a 512-value row */
#define DSA_MLA_V4_NOPE 448    /* V4 fp8 rows: fp8 NoPE values (then 64 bf16 RoPE) */
#define DSA_MLA_V4_NOPE_BYTES 512  /* V4 fp8 NoPE stream row: 448 codes, 14 E8M0, pad */

typedef enum {
    DSA_KV_BF16 = 0,
    DSA_KV_FP8_656 = 1,
    DSA_KV_BF16_D512 = 2,      /* 512 x bf16 rows (V4 prefill only) */
    DSA_KV_MXFP8 = 3,          /* MXFP8 split streams (dsa_mla_decode_mxfp8 only) */
    DSA_KV_MXFP8_V4 = 4        /* V4 fp8 rows: 448 e4m3 + 14 E8M0 + pad | 64 bf16 RoPE
                                  (dsa_mla_prefill_v4_fp8 only) */
} dsa_kv_format;

enum {
    DSA_OK = 0,
    DSA_ERR_NULL_POINTER = -1,
    DSA_ERR_BAD_SHAPE = -2,
    DSA_ERR_UNSUPPORTED = -3,
    DSA_ERR_BAD_FORMAT = -4,
    DSA_ERR_WORKSPACE = -5,
    DSA_ERR_BAD_SPLITS = -6,
    DSA_ERR_BAD_STRIDE = -7,
    DSA_ERR_HIP = -8,
    DSA_ERR_SCRATCH_LIMIT = -9
};

/*
 * Sparse MLA decode, top-k form.
 * q       : bf16 [B, s_q, H, 576] addressed by q_stride_{b,t,h} (last dim dense)
 * kv_cache: [kv_total_rows, row] in kv_format; rows are block_size-row pages,
 *           kv_stride_row elements apart (bf16 elements for DSA_KV_BF16 rows,
 *           bytes for DSA_KV_FP8_656 rows; 0 = dense rows of 576 / 656).  A
 *           row stride is at least one row, a multiple of 16 bytes and below
 *           4 GiB (else DSA_ERR_BAD_STRIDE).
 * out     : bf16 [B, s_q, H, 512] addressed by o_stride_{b,t,h}
 * lse     : fp32 [B, s_q, H] dense (may be NULL)
 * num_splits: 0 = automatic; otherwise 1..DSA_MLA_MAX_SPLITS.  With more than
 *           one split the top-k list of every query token is cut into
 *           num_splits contiguous chunks whose partial results (fp32 O and
 *           LSE, kept in the workspace) are merged by the combine kernel.
 *           A split of any length runs in one workgroup (its list is walked
 *           2048 entries at a time), so one split is always allowed.
 */
typedef struct {
    const void* q;
    int64_t q_stride_b, q_stride_t, q_stride_h;

    const void* kv_cache;
    int64_t kv_total_rows;
    int32_t kv_format;
    int32_t block_size;
    int64_t kv_batch_stride;
    int64_t kv_stride_row;       /* 0 = dense rows */

    const int32_t* block_table;
    int64_t block_table_stride;

    const int32_t* seq_lens;

    const int32_t* indices;
    int64_t idx_stride_b, idx_stride_t;

    void* out;
    int64_t o_stride_b, o_stride_t, o_stride_h;
    float* lse;

    int32_t B, s_q, H, topk;
    int32_t num_splits;
    int32_t causal;
    float sm_scale;
} dsa_mla_decode_args;

/*
 * Workspace bytes dsa_mla_decode needs for these arguments (0 when the call
 * runs unsplit).  Replaces the buffer sizing of mla_decode_plan_create,
 * opus_attn/dsa_v32/common/host.cc:151-178.
 */
int dsa_mla_decode_workspace_size(const dsa_mla_decode_args* args, size_t* bytes);

/*
 * Number of splits dsa_mla_decode uses for these arguments (resolves
 * num_splits == 0).  Pure host function.
 */
int dsa_mla_decode_num_splits(const dsa_mla_decode_args* args, int32_t* num_splits);

/*
 * Launch the decode pipeline on `stream`: the fused gather / QK / softmax /
 * PV kernel, followed by the split combine when more than one split is used.
 * Replaces mla_decode_launch_pipeline, opus_attn/dsa_v32/common/host.cc:114-138
 * (metadata -> decode -> reduce); the kernel argument block it builds carries
 * the fields of opus_mla_decode_kargs, opus_attn/dsa_v32/common/defs.h:109-131.
 */
int dsa_mla_decode(const dsa_mla_decode_args* args, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * dsa_mla_decode without a workspace and without any allocation: for callers
 * that cannot call hipMalloc (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  No counterpart in the reference.
 * The split partials go to a device scratch array the library holds on each
 * GPU for the life of the process (DSA_MLA_NOALLOC_SCRATCH_BYTES; its address
 * is looked up on a device's first call).  A call whose partials need more
 * (dsa_mla_decode_workspace_size) returns DSA_ERR_SCRATCH_LIMIT before any
 * launch; unsplit calls need none.  Calls that overlap on one GPU share its
 * scratch and race: serialise them (one stream, or events).  Results equal
 * dsa_mla_decode's on the same arguments.
 */
#define DSA_MLA_NOALLOC_SCRATCH_BYTES (16u << 20)
int dsa_mla_decode_noalloc(const dsa_mla_decode_args* args, void* stream);

/*
 * Merge split partials: partial_o fp32 [num_splits, rows, H, 512] (each split
 * normalised by its own softmax sum), partial_lse fp32 [num_splits, rows, H]
 * (natural log; -FLT_MAX marks an empty split) into out bf16 (row stride
 * o_stride_row, head stride o_stride_h, elements) and lse fp32 [rows, H]
 * (may be NULL).  rows = B * s_q.  Replaces mla_reduce_kernel,
 * opus_attn/dsa_v32/common/mla_reduce.hpp:158-184.
 */
int dsa_mla_combine(const float* partial_o, const float* partial_lse, int32_t num_splits,
                    int32_t rows, int32_t H, void* out, int64_t o_stride_row, int64_t o_stride_h,
                    float* lse, void* stream);

/*
 * Sparse MLA decode, CSR form: the argument set of the reference kernel
 * (opus_mla_decode_kargs, opus_attn/dsa_v32/common/defs.h:109-131, minus the
 * work / plan pointers the library plans itself), so a dsa_v32-style harness
 * can call it in place of mla_decode_launch_pipeline
 * (opus_attn/dsa_v32/common/host.cc:114-138).
 * q        : bf16 [B * s_q, H, 576]; query row i = b * s_q + t at
 *            q + i * stride_q_b + h * stride_q_h (elements)
 * kv       : [total_tokens, row] in kv_format; page size 1, so an index is a
 *            physical cache row.  Rows are stride_kv_page elements apart
 *            (defs.h:129, "the row stride of the latent KV tensor",
 *            opus_attn/dsa_v32/README.md:99): bf16 elements for DSA_KV_BF16
 *            rows (the reference harness passes 576), bytes for
 *            DSA_KV_FP8_656 rows; 0 = dense rows.  A row stride is at least
 *            one row, a multiple of 16 bytes and below 4 GiB.
 * kv_indptr: int32 [B + 1]; kv_indices: int32 rows.  Query token t of batch b
 *            attends kv_indices[kv_indptr[b] + p] for
 *            0 <= p < kv_indptr[b + 1] - kv_indptr[b] - (s_q - 1 - t)
 *            (count-based MTP causality, host.cc:482,526).  A row outside
 *            [0, total_tokens) is skipped; an empty range gives O = 0 and
 *            LSE = +inf (host.cc:486-489).
 * out      : bf16 [B * s_q, H, 512] at out + i * stride_o_b + h * stride_o_h
 * lse      : fp32 [B * s_q, H] dense (may be NULL)
 * max_kv_len: an upper bound of kv_indptr[b + 1] - kv_indptr[b] over b (the
 *            host cannot read the device lists; it sizes the workspace).  A
 *            query whose list is longer is not truncated silently: its O and
 *            LSE are NaN.
 * num_splits: 0 = a work plan built on the device from kv_indptr (replacing
 *            get_mla_metadata, opus_attn/dsa_v32/common/get_mla_metadata.hpp):
 *            the lists are cut into items of at most `chunk` entries sized so
 *            that all items fill about 256 workgroups (one round when there
 *            are fewer than 256 rows), whatever the spread of lengths; a row
 *            no longer than chunk is one item that writes its output
 *            directly, a longer row's items write partials that the combine
 *            merges.  The workspace then holds the plan and at most 512
 *            partial rows (H x 513 fp32 each), none when max_kv_len <= 128.
 *            DSA_MLA_SPLITS_PLANNED (-1): as 0, with the plan already in the
 *            workspace (dsa_mla_csr_plan, or an earlier call with 0), built
 *            from the same list lengths (kv_indptr) with the same B, s_q and
 *            max_kv_len: the plan is built once and reused by every layer of a
 *            decode step.  The kernels check the plan against the call: a
 *            plan built for another B, s_q or max_kv_len makes every query
 *            row's O and LSE NaN (nothing else is read or written), and a row
 *            whose list length differs from the planned one gets NaN O and
 *            LSE; a plan is never silently trusted.
 *            1..DSA_MLA_MAX_SPLITS: every row cut into num_splits equal
 *            parts (workspace: num_splits partial rows per row; none for 1).
 */
typedef struct {
    const void* q;
    const void* kv;
    void* out;
    float* lse;
    const int32_t* kv_indptr;
    const int32_t* kv_indices;
    int32_t B, s_q, H;
    int32_t total_tokens;
    int32_t stride_q_b, stride_q_h;
    int32_t stride_o_b, stride_o_h;
    int32_t stride_kv_page;      /* 0 = dense rows */
    int32_t kv_format;
    int32_t max_kv_len;
    int32_t num_splits;          /* 0 = automatic */
    float softmax_scale;
} dsa_mla_decode_csr_args;

/* Workspace bytes dsa_mla_decode_csr needs (0 for num_splits == 1). */
int dsa_mla_decode_csr_workspace_size(const dsa_mla_decode_csr_args* args, size_t* bytes);

/* Launch the CSR decode (kernel + split combine) on `stream`. */
int dsa_mla_decode_csr(const dsa_mla_decode_csr_args* args, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * Build the CSR work plan of kv_indptr (B batches, s_q query tokens each,
 * lists of at most max_kv_len entries, H heads) into `workspace` (at least
 * dsa_mla_decode_csr_workspace_size / dsa_mla_decode_mxfp8_workspace_size
 * bytes for num_splits 0), for later calls with num_splits =
 * DSA_MLA_SPLITS_PLANNED.  The counterpart of get_mla_metadata_kernel,
 * which the reference harness runs once before its timed loop
 * (opus_attn/dsa_v32/common/host.cc:266-272).  Runs on `stream`.
 */
int dsa_mla_csr_plan(const int32_t* kv_indptr, int32_t B, int32_t s_q, int32_t H, int32_t max_kv_len,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Sparse MLA decode on MXFP8 split streams, CSR form: the argument set of
 * opus_mla_decode_mxfp8_kargs (opus_attn/dsa_v32/common/defs.h:75-107, minus
 * the work / plan pointers), the reference's own "-dtype fp8" format
 * (opus_attn/dsa_v32/common/host.cc:551-697, opus_attn/dsa_v32/README.md:55-57).
 * It replaces the launch of opus_mla_decode_mxfp8_16mx8_32nx1_kernel
 * (host.cc:32-37), whose device source the reference does not ship.
 * Query row i = b * s_q + t, head h:
 *   q_nope  : fp8 e4m3fn [512] at q_nope + i * stride_q_nope_b + h * stride_q_nope_h
 *   q_scale : E8M0 [16]   at q_scale + i * stride_q_scale_b + h * stride_q_scale_h
 *   q_rope  : bf16 [64]   at q_rope + i * stride_q_rope_b + h * stride_q_rope_h
 * Cache row r (page size 1):
 *   kv_nope : fp8 e4m3fn [512] at kv_nope + r * stride_kv_nope_page
 *   kv_scale: E8M0 [16]        at kv_scale + r * stride_kv_scale_page
 *   kv_rope : bf16 [64]        at kv_rope + r * stride_kv_rope_page
 * (strides in elements of each stream: bytes for fp8 and E8M0, bf16 elements
 * for rope and out).  Value of NoPE dim d = float(e4m3(code_d)) *
 * 2^(scale[d / 32] - 127), RoPE as stored (dequant_mla_row_fp8,
 * host.cc:418-429); the kernel computes exactly these values.  Index
 * semantics, out, lse, max_kv_len and num_splits as in dsa_mla_decode_csr.
 * Alignment: the six stream pointers 16 bytes; fp8 and E8M0 strides
 * multiples of 16, bf16 strides multiples of 8, out strides of 4.
 */
typedef struct {
    const void* q_nope;
    const void* q_scale;
    const void* q_rope;
    const void* kv_nope;
    const void* kv_scale;
    const void* kv_rope;
    void* out;
    float* lse;
    const int32_t* kv_indptr;
    const int32_t* kv_indices;
    int32_t B, s_q, H;
    int32_t total_tokens;
    int32_t stride_q_nope_b, stride_q_nope_h;
    int32_t stride_q_scale_b, stride_q_scale_h;
    int32_t stride_q_rope_b, stride_q_rope_h;
    int32_t stride_o_b, stride_o_h;
    int32_t stride_kv_nope_page, stride_kv_scale_page, stride_kv_rope_page;
    int32_t max_kv_len;
    int32_t num_splits;          /* 0 = automatic */
    float softmax_scale;
} dsa_mla_decode_mxfp8_args;

/* Workspace bytes dsa_mla_decode_mxfp8 needs (0 when unsplit). */
int dsa_mla_decode_mxfp8_workspace_size(const dsa_mla_decode_mxfp8_args* args, size_t* bytes);

/* Launch the MXFP8 decode (kernel + split combine) on `stream`. */
int dsa_mla_decode_mxfp8(const dsa_mla_decode_mxfp8_args* args, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * Sparse MLA prefill (per-query top-k over one KV pool).
 * q       : bf16 [N, H, 576] addressed by q_stride_{n,h}
 * kv      : [kv_rows, row] in kv_format, rows kv_stride_row elements apart
 *           (as in dsa_mla_decode_args; 0 = dense)
 * indices : int32 [N, topk] (row stride idx_stride_n); entry j of query i is
 *           valid iff 0 <= j < kv_rows and, when causal != 0,
 *           j <= i + causal_offset
 * out     : bf16 [N, H, 512]; lse fp32 [N, H] (may be NULL)
 * num_splits: split-K over each query's list (the reference's split layout,
 *           opus_attn/dsa_v4/common/mla_prefill_split.h:7-54): 0 = automatic
 *           (more than one only when fewer than 256 workgroups, N x
 *           ceil(H / 128), would run; at least 256 list entries per split);
 *           1..DSA_MLA_MAX_SPLITS: each query's list cut into num_splits
 *           contiguous parts whose fp32 partials (O and LSE, in the
 *           workspace: num_splits x N x H x 513 floats) a combine kernel
 *           merges.  Unsplit calls need no workspace.
 * Replaces mla_v4_prefill_launch, opus_attn/dsa_v4/common/mla_v4_host.cc:28-47,
 * with the V3.2 shape (576 / 512), no attention sink, and an LSE output.
 */
typedef struct {
    const void* q;
    int64_t q_stride_n, q_stride_h;
    const void* kv;
    int64_t kv_rows;
    int64_t kv_stride_row;       /* 0 = dense rows */
    int32_t kv_format;
    const int32_t* indices;
    int64_t idx_stride_n;
    void* out;
    int64_t o_stride_n, o_stride_h;
    float* lse;
    int32_t N, H, topk;
    int32_t causal;
    int64_t causal_offset;
    float sm_scale;
    int32_t num_splits;          /* 0 = automatic */
} dsa_mla_prefill_args;

/* Workspace bytes dsa_mla_prefill needs (0 when it runs unsplit). */
int dsa_mla_prefill_workspace_size(const dsa_mla_prefill_args* args, size_t* bytes);
int dsa_mla_prefill(const dsa_mla_prefill_args* args, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * DeepSeek-V4 sparse MLA prefill: the argument set of opus_mla_v4_prefill_kargs
 * (opus_attn/dsa_v4/common/mla_v4_kargs.h:10-29), replacing
 * mla_v4_prefill_launch (opus_attn/dsa_v4/common/mla_v4_host.cc:28-47).
 * Head dim D = 512: K and V are the same 512-value bf16 row.  Query i, head h:
 *   rows = unified_kv[kv_indices_prefix[kv_indptr_prefix[i] .. kv_indptr_prefix[i+1])]
 *        followed by kv[kv_indices_extend[kv_indptr_extend[i] .. kv_indptr_extend[i+1])]
 *   s_p  = (q[i,h] . row_p) * softmax_scale
 *   P    = exp(s) / (sum exp(s) + exp(attn_sink[h]))   (no sink term when attn_sink is NULL)
 *   O    = P . rows, bf16 (mla_v4_host.cc:455-480)
 * q and out share the strides stride_qo_{n,h} (elements); cache rows are
 * stride_kv_page elements apart.  A row outside its pool is skipped; a query
 * with no rows gets O = 0 (and LSE = +inf).  lse (an addition to the
 * reference, may be NULL) is the natural log of the denominator, sink
 * included.  max_rows bounds the prefix + extend entries of any query (a
 * query with more gets NaN O and LSE, never a silently truncated attention);
 * a list of any length runs in one workgroup per split, 2048 entries at a
 * time.  total_pages and total_tokens must be below 2^30.
 * num_splits: split-K over each query's prefix-then-extend list, as the
 * reference's split prefill cuts it (opus_attn/dsa_v4/common/mla_prefill_split.h:
 * 34-44: part s of whole 32-row tiles, prefix rows first): 0 = automatic
 * (more than one only when fewer than 256 workgroups, N x ceil(H / 128),
 * would run, keeping at least 256 entries of max_rows per split); else
 * 1..DSA_MLA_MAX_SPLITS.  The splits write fp32 partials (O and LSE, no sink;
 * workspace num_splits x N x H x 513 floats, from
 * dsa_mla_prefill_v4_workspace_size) and a combine kernel merges them with
 * the sink joining the denominator once (mla_v4_host.cc:469-472).
 */
typedef struct {
    const void* q;
    const void* unified_kv;
    const void* kv;
    const float* attn_sink;
    void* out;
    float* lse;
    const int32_t* kv_indptr_prefix;
    const int32_t* kv_indices_prefix;
    const int32_t* kv_indptr_extend;
    const int32_t* kv_indices_extend;
    int32_t N, H, D;
    int32_t total_pages, total_tokens;
    int32_t stride_qo_n, stride_qo_h;
    int32_t stride_kv_page;
    int32_t max_rows;
    float softmax_scale;
    int32_t num_splits;          /* 0 = automatic (an addition to the reference kargs) */
} dsa_mla_prefill_v4_args;

/* Workspace bytes dsa_mla_prefill_v4 needs (0 when it runs unsplit). */
int dsa_mla_prefill_v4_workspace_size(const dsa_mla_prefill_v4_args* args, size_t* bytes);
int dsa_mla_prefill_v4(const dsa_mla_prefill_v4_args* args, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * DeepSeek-V4 sparse prefill on fp8 rows: the argument set of
 * opus_mla_v4_prefill_fp8_kargs (opus_attn/dsa_v4/common/mla_v4_kargs.h:31-58)
 * plus an optional LSE output and the max_rows bound.  Replaces
 * mla_v4_prefill_launch with that kargs (mla_v4_host.cc:38-47).
 * A row (and Q per head) is two streams:
 *   nope : 512 bytes = 448 e4m3fn codes, 14 E8M0 scales (one per 32 values),
 *          2 pad bytes and 48 more (the reference fills them with 0xFF)
 *   rope : 64 bf16 values
 * Value d < 448 = float(e4m3(code_d)) * 2^(scale[d / 32] - 127); values
 * 448..511 are the RoPE values (decode_dsa_row_fp8, mla_v4_host.cc:443-453).
 * K = V = the 512-value row; softmax, sink, pools, CSR lists, skipping,
 * LSE, num_splits and the workspace exactly as in dsa_mla_prefill_v4.
 * Strides in elements of each stream (bytes for nope, bf16 elements for rope
 * and out); nope pointers and strides 16-byte aligned, rope strides multiples
 * of 8, out strides of 4.  The kernel never reads the pad bytes, nor any row
 * the lists do not name.
 */
typedef struct {
    const void* q_nope;
    const void* q_rope;
    const void* unified_kv_nope;
    const void* unified_kv_rope;
    const void* kv_nope;
    const void* kv_rope;
    const float* attn_sink;
    void* out;
    float* lse;
    const int32_t* kv_indptr_prefix;
    const int32_t* kv_indices_prefix;
    const int32_t* kv_indptr_extend;
    const int32_t* kv_indices_extend;
    int32_t N, H;
    int32_t total_pages, total_tokens;
    int32_t stride_q_nope_n, stride_q_nope_h;
    int32_t stride_q_rope_n, stride_q_rope_h;
    int32_t stride_o_n, stride_o_h;
    int32_t stride_kv_nope_page, stride_kv_rope_page;
    int32_t max_rows;
    float softmax_scale;
    int32_t num_splits;          /* 0 = automatic (an addition to the reference kargs) */
} dsa_mla_prefill_v4_fp8_args;

/* Workspace bytes dsa_mla_prefill_v4_fp8 needs (0 when it runs unsplit). */
int dsa_mla_prefill_v4_fp8_workspace_size(const dsa_mla_prefill_v4_fp8_args* args, size_t* bytes);
int dsa_mla_prefill_v4_fp8(const dsa_mla_prefill_v4_fp8_args* args, void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * fp8 cache writer: quantise n_rows bf16 latent rows (576 values, row stride
 * src_stride elements) into 656-byte DSA_KV_FP8_656 rows.  Destination row
 * of source row r is dst_rows[r] (int64 physical cache row) or r when
 * dst_rows is NULL; negative destinations are skipped.  scale_g =
 * amax_g / 448 (IEEE division), code = e4m3fn(x / scale_g) with round to
 * nearest even and saturation to +-448; an all-zero group stores scale 0 and
 * zero codes.  The reference leaves cache writing to its caller
 * (opus_attn/dsa_v32/README.md:99); the codec follows float_to_fp8_e4m3,
 * opus_attn/dsa_v32/common/defs.h:11-38.
 */
int dsa_kv_quantize_fp8(const void* src_bf16, int64_t src_stride, int64_t n_rows,
                        void* dst_cache, int64_t dst_total_rows, const int64_t* dst_rows,
                        void* stream);

/* Human-readable text for a DSA_ERR_* code. */
const char* dsa_mla_strerror(int code);

/* ABI version, bumped on any change of the argument structs or of an
 * argument's meaning. */
int dsa_mla_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DSA_MLA_H_ */
