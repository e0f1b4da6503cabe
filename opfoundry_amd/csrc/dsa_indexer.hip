// dsa_indexer.hip - the DSA index scorer for gfx950 (MI355X).
//
//   score[b][t][j] = sum_h weights[b][t][h] * max(0, q[b][t][h] . k[j])
//
// (the DeepSeek-V3.2 lightning indexer's score; the reference has no indexer,
// so the contract is the library's own and is spelled out in
// include/dsa_indexer.h).  It feeds dsa_topk_indices, which selects the
// top-k positions per query token.
//
// A GEMM per sequence, Q [tokens x H_I, 128] against K [positions, 128], with
// a ReLU and a weighted sum over the index heads fused into its epilogue:
// - one workgroup (4 waves) per (sequence, group of tokens, span of 2048
//   positions); the group is 128 (token, index head) rows, so the MTP tokens of
//   a sequence (H_I = 64: two tokens) read each k row once;
// - Q stays in VGPRs as the A operand of v_mfma_f32_32x32x16_bf16 (128 rows x
//   128 dims: 128 VGPRs); k rows arrive by LDS-DMA, 128 positions (32 KB) per
//   chunk, double-buffered, and are read as the B operand;
// - wave w takes positions 32w .. 32w+31 of a chunk: 4 row blocks x 8 k-steps
//   = 32 MFMAs, then per position the weighted ReLU sum over its token's rows
//   (16 accumulator registers and one cross-half exchange per row block);
// - two workgroups per CU (73 KB of LDS each, 256 VGPRs per wave), so one's
//   epilogue and DMA issue overlap the other's MFMAs.
// Bytes per position: one 256-byte k row per sequence (all its tokens), 4-byte
// scores per token; flops: 2 * 128 per (token, head, position).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/dsa_indexer.h"
#include "dsa_lds.h"

namespace {

constexpr int IX_D = DSA_INDEXER_D;        // 128 values per index vector
constexpr int IX_NTHR = 256;
constexpr int IX_NW = IX_NTHR / 64;
constexpr int IX_QROWS = 128;              // (token, index head) rows per workgroup
constexpr int IX_CHUNK = 128;              // positions per chunk (32 per wave)
constexpr int IX_SPAN = 2048;              // positions per workgroup
constexpr int IX_KS = IX_D / 16;           // k-steps of 16
constexpr int IX_ROW = IX_D * 2;           // bytes of a k row (in LDS too: swizzled, unpadded)
constexpr int IX_BUF = IX_CHUNK * IX_ROW;  // 32 KB per chunk buffer
constexpr int IX_LPW = IX_CHUNK / 4 / IX_NW;   // LDS-DMA loads (4 rows of 256 B each) per wave per chunk

typedef __bf16 ix_bf16x8 __attribute__((ext_vector_type(8)));

struct IxParams {
    const __bf16* q;
    int64_t q_sb, q_st, q_sh;
    const float* w;
    const unsigned char* k;
    int64_t k_rows, k_row_bytes;
    const int32_t* bt;
    int64_t bt_stride;
    int32_t bs;
    int64_t k_bstride;
    const int32_t* seq_lens;
    float* scores;
    int64_t s_stride;
    int32_t s_q, n_cols, causal, tgroups;
};

// Positions j of token t of sequence b: j < min(len(b, t), n_cols).
__device__ __forceinline__ int64_t ix_len(const IxParams& p, int64_t L, int t) {
    const int64_t len = p.causal ? L - (p.s_q - 1 - t) : L;
    return min(max(len, (int64_t)0), (int64_t)p.n_cols);
}

// HI index heads per token: 128 / HI tokens per workgroup, each of the four
// 32-row blocks of Q belongs to one token.
template <int HI>
__global__ void __launch_bounds__(IX_NTHR) __attribute__((amdgpu_waves_per_eu(2, 2)))
dsa_indexer_kernel(const IxParams p) {
    constexpr int TPW = IX_QROWS / HI;
    __shared__ __attribute__((aligned(1024))) unsigned char s_k[2][IX_BUF];
    __shared__ int32_t s_rows[IX_SPAN];       // k row of each position of the span, -1: outside the cache
    __shared__ __attribute__((aligned(16))) float s_w[IX_QROWS];
    __shared__ int64_t s_len[TPW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5, r32 = lane & 31;
    const int b = blockIdx.x / p.tgroups;
    const int t0 = (blockIdx.x - b * p.tgroups) * TPW;
    const int ntok = min(TPW, p.s_q - t0);
    const int64_t span0 = (int64_t)blockIdx.y * IX_SPAN;
    const int64_t L = p.seq_lens[b];
    // the group's longest list: its last token's (the lists grow with t)
    const int64_t lmax = ix_len(p, L, t0 + ntok - 1);
    if (span0 >= lmax) return;                 // the whole workgroup, before any barrier
    const int nspan = (int)min((int64_t)IX_SPAN, lmax - span0);
    const int nchunks = (nspan + IX_CHUNK - 1) / IX_CHUNK;
    const bool any_rows = p.k_rows > 0;

    // ---- Q (A operand): lane (r32, hi) holds rows 32qb + r32, dims 16ks + 8hi .. +7 ----
    u32x4 qf[4][IX_KS];
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) {
        const int qrow = 32 * qb + r32;
        const int tl = min(qrow / HI, ntok - 1);   // rows of a missing token: a copy, never stored
        const __bf16* qp = p.q + (int64_t)b * p.q_sb + (int64_t)(t0 + tl) * p.q_st + (int64_t)(qrow % HI) * p.q_sh + 8 * hi;
#pragma unroll
        for (int ks = 0; ks < IX_KS; ++ks) qf[qb][ks] = *reinterpret_cast<const u32x4*>(qp + 16 * ks);
    }
    if (tid < IX_QROWS) {
        const int tl = min(tid / HI, ntok - 1);
        s_w[tid] = p.w[((int64_t)b * p.s_q + t0 + tl) * HI + tid % HI];
    }
    if (tid < TPW) s_len[tid] = tid < ntok ? ix_len(p, L, t0 + tid) : 0;
    // ---- the span's k rows (the dsa_mla_decode top-k rules) ----
#pragma unroll
    for (int e = 0; e < IX_SPAN / IX_NTHR; ++e) {
        const int rl = tid * (IX_SPAN / IX_NTHR) + e;
        int32_t row = -1;
        if (rl < nspan) {
            const int64_t j = span0 + rl;
            int64_t phys;
            if (p.bt) {
                const int32_t blk = p.bt[(int64_t)b * p.bt_stride + j / p.bs];
                phys = (int64_t)blk * p.bs + j % p.bs;
            } else {
                phys = (int64_t)b * p.k_bstride + j;
            }
            if (phys >= 0 && phys < p.k_rows) row = (int32_t)phys;
        }
        s_rows[rl] = row;
    }
    // Q, weights and rows complete: in the chunk loop the only vector-memory
    // loads are the LDS-DMA k rows, counted explicitly.
    wait_vm<0>();
    __syncthreads();

    // chunk c -> buffer nb: wave w loads rows 4(8w + i) .. +3 of the chunk (16
    // lanes x 16 bytes per row); a row's 16-byte piece d is stored at slot
    // d ^ (row & 15), so the B-operand reads below (32 rows, one piece each)
    // spread over the banks.  A row outside the cache is read from row 0 and
    // scored -inf.
    auto issue = [&](int c, int nb) {
#pragma unroll
        for (int i = 0; i < IX_LPW; ++i) {
            const int rc = 4 * (IX_LPW * wave + i) + (lane >> 4);    // row within the chunk
            const int32_t row = max(s_rows[c * IX_CHUNK + rc], 0);
            const int piece = (lane & 15) ^ (rc & 15);
            lds_dma16(p.k + (int64_t)row * p.k_row_bytes + 16 * piece,
                      (lds_ptr)s_k[nb] + 4 * (IX_LPW * wave + i) * IX_ROW);
        }
    };
    if (any_rows) issue(0, 0);
    for (int c = 0; c < nchunks; ++c) {
        if (any_rows) {
            if (c + 1 < nchunks) {
                // buffer (c+1)&1 held chunk c-1, done with at the last barrier
                issue(c + 1, (c + 1) & 1);
                wait_vm<IX_LPW>();         // chunk c landed (this wave's loads)
            } else {
                wait_vm<0>();
            }
        }
        tile_barrier();                    // every wave's loads of chunk c landed
        f32x16 acc[4];
#pragma unroll
        for (int qb = 0; qb < 4; ++qb) acc[qb] = f32x16{};
        if (any_rows) {
            // B operand: lane (r32, hi) holds k row 32w + r32, dims 16ks + 8hi .. +7
            const int rc = 32 * wave + r32;
            const lds_cptr kr = (lds_cptr)s_k[c & 1] + rc * IX_ROW;
#pragma unroll
            for (int ks = 0; ks < IX_KS; ++ks) {
                const u32x4 kf = lds_ld<u32x4>(kr + 16 * ((2 * ks + hi) ^ (rc & 15)));
#pragma unroll
                for (int qb = 0; qb < 4; ++qb)
                    acc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(ix_bf16x8, qf[qb][ks]),
                                                                      __builtin_bit_cast(ix_bf16x8, kf), acc[qb],
                                                                      0, 0, 0);
            }
        }
        // ---- epilogue: lane (r32, hi) has position 32w + r32 of the chunk, and
        // in register r of row block qb the row 32qb + 8(r/4) + 4hi + r%4 ----
        const int pl = c * IX_CHUNK + 32 * wave + r32;    // position within the span
        const int64_t j = span0 + pl;
        const bool bad = s_rows[pl] < 0;
        // token tk: row blocks tk * HI / 32 .. (tk + 1) * HI / 32 - 1, one token
        // at a time (few values live beside Q and the accumulators)
#pragma unroll
        for (int tk = 0; tk < TPW; ++tk) {
            float part = 0.0f;
#pragma unroll
            for (int qb = tk * HI / 32; qb < (tk + 1) * HI / 32; ++qb) {
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const f32x4 wv = lds_ld<f32x4>((lds_cptr)s_w + 4 * (32 * qb + 8 * r4 + 4 * hi));
#pragma unroll
                    for (int e = 0; e < 4; ++e) part += wv[e] * fmaxf(acc[qb][4 * r4 + e], 0.0f);
                }
            }
            part += __shfl_xor(part, 32, 64);
            // token tk's score leaves through the lanes of half (tk & 1)
            if ((tk & 1) == hi && tk < ntok && j < s_len[tk])
                p.scores[((int64_t)b * p.s_q + t0 + tk) * p.s_stride + j] = bad ? -INFINITY : part;
        }
        tile_barrier();                    // every wave done with buffer c&1
    }
}

template <int HI>
int launch_ix(const IxParams& p, int B, int ycount, hipStream_t st) {
    dim3 grid((unsigned)((int64_t)B * p.tgroups), (unsigned)ycount), block(IX_NTHR);
    hipLaunchKernelGGL(dsa_indexer_kernel<HI>, grid, block, 0, st, p);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

}  // namespace

extern "C" int dsa_indexer_scores(const dsa_indexer_args* a, void* stream) {
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->B < 0 || a->s_q <= 0 || a->n_cols < 0 || a->k_total_rows < 0 || a->k_total_rows > INT32_MAX)
        return DSA_ERR_BAD_SHAPE;
    if (a->H_I != 32 && a->H_I != 64 && a->H_I != 128) return DSA_ERR_UNSUPPORTED;
    if (a->block_table && a->block_size <= 0) return DSA_ERR_BAD_SHAPE;
    const int64_t k_stride = a->k_stride_row ? a->k_stride_row : DSA_INDEXER_D;
    if (k_stride < DSA_INDEXER_D || (k_stride % 8)) return DSA_ERR_BAD_STRIDE;
    if (a->score_stride < a->n_cols) return DSA_ERR_BAD_STRIDE;
    const int tpw = 128 / a->H_I;
    const int tgroups = (a->s_q + tpw - 1) / tpw;
    if ((int64_t)a->B * tgroups > INT32_MAX) return DSA_ERR_BAD_SHAPE;
    if (a->B == 0 || a->n_cols == 0) return DSA_OK;
    if (!a->q || !a->weights || !a->seq_lens || !a->scores || (a->k_total_rows > 0 && !a->k_cache))
        return DSA_ERR_NULL_POINTER;
    if ((a->q_stride_b % 8) || (a->q_stride_t % 8) || (a->q_stride_h % 8) || ((uintptr_t)a->q & 15) ||
        ((uintptr_t)a->k_cache & 15) || ((uintptr_t)a->scores & 3))
        return DSA_ERR_BAD_STRIDE;
    IxParams p{};
    p.q = (const __bf16*)a->q;
    p.q_sb = a->q_stride_b; p.q_st = a->q_stride_t; p.q_sh = a->q_stride_h;
    p.w = a->weights;
    p.k = (const unsigned char*)a->k_cache;
    p.k_rows = a->k_total_rows;
    p.k_row_bytes = 2 * k_stride;
    p.bt = a->block_table;
    p.bt_stride = a->block_table_stride;
    p.bs = a->block_table ? a->block_size : 1;
    p.k_bstride = a->k_batch_stride;
    p.seq_lens = a->seq_lens;
    p.scores = a->scores;
    p.s_stride = a->score_stride;
    p.s_q = a->s_q; p.n_cols = a->n_cols; p.causal = a->causal ? 1 : 0; p.tgroups = tgroups;
    const int ycount = (a->n_cols + IX_SPAN - 1) / IX_SPAN;
    hipStream_t st = (hipStream_t)stream;
    if (a->H_I == 32) return launch_ix<32>(p, a->B, ycount, st);
    if (a->H_I == 64) return launch_ix<64>(p, a->B, ycount, st);
    return launch_ix<128>(p, a->B, ycount, st);
}
