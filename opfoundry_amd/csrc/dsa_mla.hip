// dsa_mla.hip - gfx950 (MI355X) sparse MLA decode / prefill kernels and the
// C ABI declared in include/dsa_mla.h.
//
// One workgroup handles one (query token, top-k split): 4 waves x 32 heads =
// 128 heads, so every gathered latent row is read from HBM once and used by
// all heads.  Per tile of 32 rows:
//   gather   rows -> LDS ring with 16-byte LDS-DMA loads (global_load_lds);
//            fp8 rows land raw and are dequantised cooperatively into the
//            bf16 tile (e4m3 -> fp32 exact, times the per-128 scale, -> bf16)
//   QK^T     S^T[32 rows x 32 heads] = K Q^T with 32x32x16 bf16 MFMA, Q held
//            in registers for the whole workgroup lifetime
//   softmax  exp2-domain softmax numerators against a fixed per-head
//            reference max (no accumulator rescale in the loop); the
//            per-head max is a lane-local max plus one cross-half exchange
//   PV       O^T[512 x 32 heads] += V^T P^T, V^T read with ds_read_b64_tr_b16
//            straight from the row-major tile, P^T taken from the S^T
//            accumulator registers without any shuffle
// The decode kernel design follows the reference's one-workgroup-per-work-item
// structure (opus_attn/dsa_v32/gfx950/mla_decode_a16w16_32mxt_32nx1_template.hpp:
// 916-1132) but is written from scratch for stock hipcc: no OPUS, no pinned
// registers, 32x32 MFMA tiles, compacted index lists and a top-k index form.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>
#include <algorithm>

#include "../../include/dsa_mla.h"

namespace {

constexpr int D_QK = DSA_MLA_D_QK;
constexpr int D_NOPE = DSA_MLA_D_NOPE;
constexpr int D_ROPE = DSA_MLA_D_ROPE;
constexpr int D_VO = DSA_MLA_D_VO;
constexpr int HEADS = 128;                 // heads per workgroup (4 waves x 32)
constexpr int NWAVE = 4;
constexpr int NTHR = NWAVE * 64;
constexpr int TILE = 32;                   // latent rows per tile
constexpr int MAX_CHUNK = 2048;            // top-k entries one workgroup can take
constexpr int ROWB = D_QK * 2;             // bf16 cache row bytes (1152)
// bf16 tile in LDS: NoPE rows at a 1040-byte stride (65 16-byte chunks, so the
// 32 rows a K fragment touches fall in distinct bank groups), then the RoPE
// block, 32 rows x 128 B with the chunks of row r XOR-swizzled by row_swz(r).
constexpr int NOPE_STRIDE = 2 * D_NOPE + 16;            // 1040
constexpr int ROPE_BASE = TILE * NOPE_STRIDE;          // 33280
constexpr int ROPE_STRIDE = 2 * D_ROPE;                // 128
constexpr int SLOT_BF16 = ROPE_BASE + TILE * ROPE_STRIDE;  // 37376
constexpr int LD_BF16_PER_WAVE = TILE / NWAVE + 1;     // 8 NoPE rows + 1 RoPE block (9)
constexpr int FP8_CH = DSA_MLA_FP8_ROW_BYTES / 16;  // 16-byte chunks per fp8 row (41)
constexpr int LD_FP8_PER_WAVE = 6;                   // >= ceil(32*41/64/4), uniform per wave
constexpr int SLOT_FP8 = LD_FP8_PER_WAVE * NWAVE * 1024;  // raw fp8 tile incl. pad (24576 B)
constexpr int NS_BF16 = 3;                 // bf16-path ring depth
constexpr int NS_RAW = 3;                  // fp8-path raw ring depth (+1 bf16 tile)
constexpr int QK_REG = 28;                 // k-steps whose Q fragments live in registers (dims 0..447)
constexpr int QL_DIMS = D_QK - 16 * QK_REG; // Q dims kept in LDS instead (448..575: 128)
constexpr int QR_STRIDE = 2 * QL_DIMS + 16; // LDS bytes per head of that Q block (272)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.69314718055994531f;
constexpr float RESTART_TAU = 64.0f;       // max growth of p over the reference max (log2 units)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

#define LDS_AS __attribute__((address_space(3)))
#define GLB_AS __attribute__((address_space(1)))

// 32-bit LDS addresses: every LDS access in the kernels goes through these
// (a generic pointer would cost a 64-bit VGPR pair per address).
typedef LDS_AS unsigned char* lds_ptr;
typedef const LDS_AS unsigned char* lds_cptr;

// 1152 zero bytes: invalid tile slots gather this row, so masked slots always
// hold finite K and V = 0 (a poisoned cache row can never leak in as NaN * 0).
__device__ __attribute__((aligned(16))) unsigned char g_zero_row[ROWB];

// Swizzle of the 8 RoPE chunks of row r: chunk c lives at position c ^ x(r).
// x is a bijection on every 8 consecutive rows and on the even / odd rows of
// every 16, so 32 rows reading the same chunk spread over all bank groups of
// a 32- or 64-bank LDS even though the RoPE rows are only 128 B apart.
__device__ __forceinline__ int row_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

struct FwdParams {
    const __bf16* q;
    int64_t q_sb, q_st, q_sh;
    const unsigned char* kv;
    int64_t kv_total_rows;
    int64_t kv_batch_stride;
    const int32_t* block_table;
    int64_t bt_stride;
    int32_t block_size;
    int32_t bs_shift;            // log2(block_size) when a power of two, else -1
    const int32_t* seq_lens;     // NULL: every query uses seq_len_default
    int64_t seq_len_default;
    const int32_t* indices;
    int64_t idx_sb, idx_st;
    __bf16* out;
    int64_t o_sb, o_st, o_sh;
    float* lse;
    float* part_o;               // [splits][B*s_q][128][512] fp32, NULL when unsplit
    float* part_lse;             // [splits][B*s_q][128]
    int32_t B, s_q, topk, chunk;
    int32_t causal;              // 1: decode rule  j <= L - s_q + t
                                 // 2: prefill rule j <= b + causal_offset
    int64_t causal_offset;
    float scale_log2;            // sm_scale * log2(e)
};

__device__ __forceinline__ void wait_vmcnt_le(int n) {
    // s_waitcnt vmcnt(n), expcnt/lgkmcnt left at their maxima (gfx9 encoding).
    switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    case 9: __builtin_amdgcn_s_waitcnt(0x0F79); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
    case 18: __builtin_amdgcn_s_waitcnt(0x4F72); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    }
}

// Keep an MFMA accumulator tile in AGPRs (an empty asm with an AGPR operand):
// the O accumulators stay there for the whole kernel and only the rare
// rescale moves them through VGPRs.
__device__ __forceinline__ void pin_acc(f32x16& v) { asm volatile("" : "+a"(v)); }
// Keep a tile the VALU reads next (the score accumulator) in VGPRs.
__device__ __forceinline__ void pin_vgpr(f32x16& v) { asm volatile("" : "+v"(v)); }

// Opaque copy: stops the compiler from hoisting per-lane address math out of
// the tile loop (which would pin dozens of loop-invariant VGPRs).
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// 16-byte LDS-DMA load: lane l's 16 bytes from gsrc land at lds_wave_base +
// 16*l.  Issued through inline asm so the compiler neither waits on it at the
// next LDS read nor folds it into its own vmcnt accounting: the tile loop
// tracks these loads itself with explicit s_waitcnt vmcnt(N) (wait_vmcnt_le),
// and no other vector-memory load is issued inside the loop.
__device__ __forceinline__ void lds_dma16(const void* gsrc, lds_ptr lds_wave_base) {
    const unsigned m0v = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_wave_base);
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off"
        :
        : "s"(m0v), "v"(gsrc)
        : "memory", "m0");
}

// Workgroup barrier for the tile loop: LDS writes of this wave complete, then
// s_barrier.  Unlike __syncthreads() it does not drain vector memory, so the
// LDS-DMA gathers of later tiles stay in flight across it.
__device__ __forceinline__ void tile_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ bf16x8 lds_read_b128(lds_cptr p) {
    return *reinterpret_cast<const LDS_AS bf16x8*>(p);
}

__device__ __forceinline__ s16x4 lds_read_tr16(lds_cptr p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS s16x4*)(p));
}

// Physical cache row of logical position j of query (b, t); -1 if invalid.
__device__ __forceinline__ int64_t resolve_row(const FwdParams& p, int b, int64_t jmax, int32_t j) {
    if (j < 0 || (int64_t)j >= jmax) return -1;
    int64_t row;
    if (p.block_table) {
        const int32_t blk_i = p.bs_shift >= 0 ? (j >> p.bs_shift) : (j / p.block_size);
        const int32_t in_blk = p.bs_shift >= 0 ? (j & (p.block_size - 1)) : (j % p.block_size);
        const int32_t blk = p.block_table[(int64_t)b * p.bt_stride + blk_i];
        row = (int64_t)blk * p.block_size + in_blk;
    } else {
        row = (int64_t)b * p.kv_batch_stride + j;
    }
    if (row < 0 || row >= p.kv_total_rows) return -1;
    return row;
}

// ---------------------------------------------------------------------------
// Fused sparse-MLA forward: one workgroup per (query token, split).
// grid = (B, s_q, num_splits), block = 256.
// ---------------------------------------------------------------------------
template <int FMT>
__global__ void __launch_bounds__(NTHR) __attribute__((amdgpu_waves_per_eu(1, 1)))
dsa_mla_fwd_kernel(const FwdParams p) {
    constexpr int NS = FMT == DSA_KV_BF16 ? NS_BF16 : NS_RAW;
    constexpr int RAW_SLOT = FMT == DSA_KV_BF16 ? SLOT_BF16 : SLOT_FP8;
    __shared__ __attribute__((aligned(1024))) unsigned char s_raw[NS * RAW_SLOT];
    // fp8 only: the dequantised bf16 tile.  One buffer suffices: the tile
    // barrier at the top of each iteration orders compute(it-1) before
    // dequant(it).
    __shared__ __attribute__((aligned(1024))) unsigned char s_bf[FMT == DSA_KV_BF16 ? 16 : SLOT_BF16];
    // Tail of Q (dims 448..575), [128 heads][128] bf16 with a 272-byte head
    // stride (the 16-byte pad spreads 16 consecutive heads over distinct bank
    // groups).  Holding it here instead of in registers leaves the tile loop
    // enough VGPRs to run without spills.
    __shared__ __attribute__((aligned(16))) unsigned char s_qr[HEADS * QR_STRIDE];
    __shared__ int32_t s_rows[MAX_CHUNK];
    __shared__ int s_wsum[NWAVE];
    __shared__ int s_restart;
    const lds_ptr L_raw = (lds_ptr)s_raw;
    const lds_ptr L_bf = (lds_ptr)s_bf;
    const lds_ptr L_qr = (lds_ptr)s_qr;

    const int b = blockIdx.x, t = blockIdx.y, split = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_restart = 0;

    // ---- 1. resolve this split's index chunk into a compacted row list ----
    const int k0 = split * p.chunk;
    const int k1 = min(k0 + p.chunk, p.topk);
    int64_t L = p.seq_lens ? (int64_t)p.seq_lens[b] : p.seq_len_default;
    int64_t jmax = L;
    if (p.causal == 1) jmax = min(L, L - p.s_q + t + 1);
    else if (p.causal == 2) jmax = min(L, (int64_t)b + p.causal_offset + 1);
    const int32_t* idx = p.indices + (int64_t)b * p.idx_sb + (int64_t)t * p.idx_st;

    constexpr int PER_T = MAX_CHUNK / NTHR;  // 8 entries per thread
    int32_t rows_local[PER_T];
    int cnt = 0;
    {
        int32_t jv[PER_T];
#pragma unroll
        for (int e = 0; e < PER_T; ++e) {
            const int k = k0 + tid * PER_T + e;
            jv[e] = k < k1 ? idx[k] : -1;
        }
#pragma unroll
        for (int e = 0; e < PER_T; ++e) {
            rows_local[e] = (int32_t)resolve_row(p, b, jmax, jv[e]);
            cnt += rows_local[e] >= 0 ? 1 : 0;
        }
    }
    // block-wide exclusive scan of cnt
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    int wbase = 0, n_valid = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
        const int s = s_wsum[w];
        wbase += w < wave ? s : 0;
        n_valid += s;
    }
    {
        int pos = wbase + incl - cnt;
#pragma unroll
        for (int e = 0; e < PER_T; ++e)
            if (rows_local[e] >= 0) s_rows[pos++] = rows_local[e];
    }
    __syncthreads();
    const int ntiles = (n_valid + TILE - 1) / TILE;

    // ---- 2. Q fragments: B operand of S^T = K Q^T, lane -> head lane%32 ----
    const int h32 = lane & 31, hi = lane >> 5;
    const int head = wave * 32 + h32;
    bf16x8 qf[QK_REG];
    {
        const __bf16* qp = p.q + (int64_t)b * p.q_sb + (int64_t)t * p.q_st + (int64_t)head * p.q_sh + 8 * hi;
#pragma unroll
        for (int ks = 0; ks < QK_REG; ++ks)
            qf[ks] = *reinterpret_cast<const bf16x8*>(qp + 16 * ks);
        // Q tail -> LDS: 128 heads x 16 chunks of 16 B, 8 per thread
        const __bf16* qb = p.q + (int64_t)b * p.q_sb + (int64_t)t * p.q_st + 16 * QK_REG;
#pragma unroll
        for (int i = 0; i < (HEADS * QL_DIMS / 8) / NTHR; ++i) {
            const int u = tid + NTHR * i;
            const int hh = u / (QL_DIMS / 8), c = u % (QL_DIMS / 8);
            *reinterpret_cast<LDS_AS u32x4*>(L_qr + hh * QR_STRIDE + 16 * c) =
                *reinterpret_cast<const u32x4*>(qb + (int64_t)hh * p.q_sh + 8 * c);
        }
    }
    // Q fragments complete before the tile loop: inside the loop the only
    // vector-memory loads are the LDS-DMA gathers counted by wait_vmcnt_le.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    lds_cptr qr_lane = L_qr + head * QR_STRIDE + 16 * hi;

    // ---- gather issue: tile `it` into ring slot `slot` ----
    auto issue_tile = [&](int it, int slot) {
        const int ln = opaque(lane);
        if constexpr (FMT == DSA_KV_BF16) {
            lds_ptr slot_base = L_raw + slot * RAW_SLOT;
            // NoPE: one wave instruction per row, lane = 16-byte chunk
#pragma unroll
            for (int i = 0; i < TILE / NWAVE; ++i) {
                const int r = (TILE / NWAVE) * wave + i;
                const int row = it * TILE + r;
                const unsigned char* src = row < n_valid ? p.kv + (int64_t)s_rows[row] * ROWB : g_zero_row;
                lds_dma16(src + 16 * ln, slot_base + r * NOPE_STRIDE);
            }
            // RoPE: rows 8w..8w+7, lane -> (row 8w + lane/8, LDS position lane%8)
            {
                const int r = (TILE / NWAVE) * wave + (ln >> 3);
                const int row = it * TILE + r;
                const int c = (ln & 7) ^ row_swz(r);  // global RoPE chunk stored at position lane%8
                const unsigned char* src = row < n_valid ? p.kv + (int64_t)s_rows[row] * ROWB : g_zero_row;
                lds_dma16(src + 2 * D_NOPE + 16 * c, slot_base + ROPE_BASE + (TILE / NWAVE) * wave * ROPE_STRIDE);
            }
        } else {
#pragma unroll
            for (int i = 0; i < LD_FP8_PER_WAVE; ++i) {
                const int k = wave + NWAVE * i;
                const int pch = 64 * k + ln;
                const int r = pch / FP8_CH, c = pch - r * FP8_CH;
                const int slot_row = it * TILE + r;
                const unsigned char* src = (r < TILE && slot_row < n_valid)
                    ? p.kv + (int64_t)s_rows[slot_row] * DSA_MLA_FP8_ROW_BYTES + 16 * c
                    : g_zero_row;
                lds_dma16(src, L_raw + slot * RAW_SLOT + 1024 * k);
            }
        }
    };

    constexpr int LOADS_PER_TILE = FMT == DSA_KV_BF16 ? LD_BF16_PER_WAVE : LD_FP8_PER_WAVE;

    // ---- fp8: dequantise raw slot -> bf16 tile (cooperative) ----
    auto dequant_tile = [&](lds_cptr raw, lds_ptr dst) {
        // NoPE: 32 rows x 32 groups of 16 codes = 1024 units, 4 per thread.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = tid + NTHR * i;
            const int r = u >> 5, q16 = u & 31;
            lds_cptr rr = raw + r * DSA_MLA_FP8_ROW_BYTES;
            const u32x4 codes = *reinterpret_cast<const LDS_AS u32x4*>(rr + 16 * q16);
            const float sc = *reinterpret_cast<const LDS_AS float*>(rr + D_NOPE + 4 * (q16 >> 3));
            u32x4 lo, hi2;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes[w], false);
                const f32x2 c2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes[w], true);
                const bf16x2 ba = __builtin_convertvector(a * sc, bf16x2);
                const bf16x2 bc = __builtin_convertvector(c2 * sc, bf16x2);
                const unsigned ua = __builtin_bit_cast(unsigned, ba);
                const unsigned uc = __builtin_bit_cast(unsigned, bc);
                if (w < 2) { lo[2 * w] = ua; lo[2 * w + 1] = uc; }
                else { hi2[2 * (w - 2)] = ua; hi2[2 * (w - 2) + 1] = uc; }
            }
            lds_ptr drow = dst + r * NOPE_STRIDE + 32 * q16;  // bf16 chunks 2q16, 2q16+1
            *reinterpret_cast<LDS_AS u32x4*>(drow) = lo;
            *reinterpret_cast<LDS_AS u32x4*>(drow + 16) = hi2;
        }
        // RoPE: 32 rows x 8 chunks of 8 bf16 = 256 units, 1 per thread.
        {
            const int r = tid >> 3, c = tid & 7;
            const u32x4 v = *reinterpret_cast<const LDS_AS u32x4*>(
                raw + r * DSA_MLA_FP8_ROW_BYTES + 528 + 16 * c);
            *reinterpret_cast<LDS_AS u32x4*>(
                dst + ROPE_BASE + r * ROPE_STRIDE + 16 * (c ^ row_swz(r))) = v;
        }
    };

    // ---- online softmax with a fixed reference max ----
    // p = exp2(s - m_ref) with m_ref fixed for the whole pass (the first tile's
    // max per head), so the O accumulators are never rescaled inside the tile
    // loop.  p may grow up to 2^RESTART_TAU (fp32 / bf16 have the range and
    // the result is scale-invariant).  A tile whose max exceeds m_ref + TAU
    // raises s_restart; after the pass the workgroup restarts from tile 0 with
    // m_ref = the largest score seen, discarding the partial sums.  For inputs whose
    // scores stay within 2^64 of the first tile's maximum this never happens.
    f32x16 o[D_VO / 32];
    float m_ref = -INFINITY, m_seen = -INFINITY, l_lane = 0.0f;

    for (;;) {
#pragma unroll
        for (int mb = 0; mb < D_VO / 32; ++mb) {
            o[mb] = f32x16{};
            pin_acc(o[mb]);
        }
#pragma unroll
        for (int s = 0; s < NS - 1; ++s)
            if (s < ntiles) issue_tile(s, s);

        for (int it = 0; it < ntiles; ++it) {
            // tile `it` must have landed; newer tiles may stay in flight
            if (it + NS - 2 < ntiles) wait_vmcnt_le(LOADS_PER_TILE * (NS - 2));
            else wait_vmcnt_le(0);
            tile_barrier();
            if (it + NS - 1 < ntiles) issue_tile(it + NS - 1, (it + NS - 1) % NS);

            lds_cptr kt;
            if constexpr (FMT == DSA_KV_BF16) {
                kt = L_raw + (it % NS) * RAW_SLOT;
            } else {
                lds_ptr dst = L_bf;
                dequant_tile(L_raw + (it % NS) * RAW_SLOT, dst);
                tile_barrier();
                kt = dst;
            }

            // ---- S^T = K Q^T (32 rows x 32 heads) ----
            __builtin_amdgcn_sched_barrier(0);
            f32x16 sacc = f32x16{};
            {
                // K fragment of k-step ks: row lane%32, 16-byte chunk 2ks+hi.
                // NoPE steps: one base + immediate; RoPE steps: swizzled chunk.
                const int r = lane & 31;
                lds_cptr kb = kt + r * NOPE_STRIDE + 16 * hi;
                lds_cptr kr = kt + ROPE_BASE + r * ROPE_STRIDE;
                const int sw = row_swz(r);
#pragma unroll
                for (int ks = 0; ks < D_QK / 16; ++ks) {
                    constexpr int KS_NOPE = D_NOPE / 16;
                    const bf16x8 a0 = ks < KS_NOPE ? lds_read_b128(kb + 32 * ks)
                                                   : lds_read_b128(kr + 16 * ((2 * (ks - KS_NOPE) + hi) ^ sw));
                    const bf16x8 qv = ks < QK_REG ? qf[ks < QK_REG ? ks : 0] : lds_read_b128(qr_lane + 32 * (ks - QK_REG));
                    sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qv, sacc, 0, 0, 0);
                    // (accumulator placement left to the register allocator)
                }
                // issue order: K-fragment reads run QK_PF ahead of the MFMAs
                // (the last D_ROPE/16 steps also read their Q fragment)
                constexpr int NK = D_QK / 16, QK_PF = 3;
                __builtin_amdgcn_sched_group_barrier(0x100, QK_PF, 0);
#pragma unroll
                for (int i = 0; i < QK_REG - QK_PF; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
#pragma unroll
                for (int i = QK_REG - QK_PF; i < NK - QK_PF; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                }
#pragma unroll
                for (int i = 0; i < QK_PF; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);

            // ---- softmax numerators for this tile ----
            // lane (hi, h32), reg r holds row 8*(r/4) + 4*hi + r%4 of head h32
            float mx = -INFINITY;
            const int row0 = it * TILE;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 8 * (r >> 2) + 4 * hi + (r & 3);
                sacc[r] = row0 + row < n_valid ? sacc[r] * p.scale_log2 : -INFINITY;
                mx = fmaxf(mx, sacc[r]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            m_seen = fmaxf(m_seen, mx);
            if (m_ref == -INFINITY) m_ref = mx;
            if (__builtin_amdgcn_ballot_w64(mx > m_ref + RESTART_TAU) != 0 && lane == 0) s_restart = 1;
            const float m_use = m_ref == -INFINITY ? 0.0f : m_ref;
            f32x8 pv0, pv1;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float e = __builtin_amdgcn_exp2f(sacc[r] - m_use);
                l_lane += e;
                if (r < 8) pv0[r] = e; else pv1[r - 8] = e;
            }
            if (ntiles == 1) {
                // Every valid row is in this tile: normalise by the exact sum before the
                // bf16 rounding of P, the order the reference uses (host.cc:448-451).
                const float lt = l_lane + __shfl_xor(l_lane, 32, 64);
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    pv0[r] = pv0[r] / lt;
                    pv1[r] = pv1[r] / lt;
                }
            }
            const bf16x8 pb0 = __builtin_convertvector(pv0, bf16x8);
            const bf16x8 pb1 = __builtin_convertvector(pv1, bf16x8);

            // ---- O^T += V^T P^T ----
            __builtin_amdgcn_sched_barrier(0);
            {
                // Transposed read of rows R..R+3, columns d0..d0+15 (16-lane group):
                // lane 4*rr+pp addresses row R+rr, columns d0+4pp..+3.  This wave
                // needs R = 8a + 4hi (a = 2u, 2u+1) and d0 = 32mb + 16dh, so one
                // per-lane base plus immediates covers every read.
                const int g16 = lane >> 4, i16 = lane & 15;
                const int rr = i16 >> 2, pp = i16 & 3;
                const int dh = g16 & 1;
                lds_cptr vb = kt + (4 * hi + rr) * NOPE_STRIDE + 32 * dh + 8 * pp;
#pragma unroll
                for (int mb = 0; mb < D_VO / 32; ++mb) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const s16x4 va = lds_read_tr16(vb + 16 * u * NOPE_STRIDE + 64 * mb);
                        const s16x4 vv = lds_read_tr16(vb + (16 * u + 8) * NOPE_STRIDE + 64 * mb);
                        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(va, vv, 0, 1, 2, 3, 4, 5, 6, 7));
                        o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, u == 0 ? pb0 : pb1, o[mb], 0, 0, 0);
                        pin_acc(o[mb]);
                    }
                }
                // issue order: two transposed reads per MFMA, PV_PF fragments ahead
                constexpr int NM = 2 * (D_VO / 32), PV_PF = 2;
                __builtin_amdgcn_sched_group_barrier(0x100, 2 * PV_PF, 0);
#pragma unroll
                for (int i = 0; i < NM - PV_PF; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                }
#pragma unroll
                for (int i = 0; i < PV_PF; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // drain in-flight gathers before the ring can be reused or left
        wait_vmcnt_le(0);
        tile_barrier();
        if (!s_restart) break;
        tile_barrier();              // every wave has seen the flag
        if (tid == 0) s_restart = 0;  // visible after the next tile barrier
        m_ref = m_seen;
        l_lane = 0.0f;
    }

    // ---- epilogue ----
    const float l = l_lane + __shfl_xor(l_lane, 32, 64);
    const bool has = l > 0.0f;
    const float inv = has ? (ntiles == 1 ? 1.0f : 1.0f / l) : 0.0f;  // one tile: P was normalised
    const int64_t qrow = (int64_t)b * p.s_q + t;
    if (p.part_o == nullptr) {
        __bf16* op = p.out + (int64_t)b * p.o_sb + (int64_t)t * p.o_st + (int64_t)head * p.o_sh;
#pragma unroll
        for (int mb = 0; mb < D_VO / 32; ++mb) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v4 = {o[mb][4 * g] * inv, o[mb][4 * g + 1] * inv, o[mb][4 * g + 2] * inv,
                                  o[mb][4 * g + 3] * inv};
                typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
                const bf16x4 bv = __builtin_convertvector(v4, bf16x4);
                *reinterpret_cast<u32x2*>(op + 32 * mb + 8 * g + 4 * hi) = __builtin_bit_cast(u32x2, bv);
            }
        }
        if (p.lse && hi == 0)
            p.lse[qrow * HEADS + head] = has ? (m_ref + __builtin_amdgcn_logf(l)) * LN2 : INFINITY;
    } else {
        const int64_t prow = ((int64_t)split * p.B * p.s_q + qrow) * HEADS + head;
        float* op = p.part_o + prow * D_VO;
#pragma unroll
        for (int mb = 0; mb < D_VO / 32; ++mb) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v4 = {o[mb][4 * g] * inv, o[mb][4 * g + 1] * inv, o[mb][4 * g + 2] * inv,
                                  o[mb][4 * g + 3] * inv};
                *reinterpret_cast<f32x4*>(op + 32 * mb + 8 * g + 4 * hi) = v4;
            }
        }
        if (hi == 0) p.part_lse[prow] = has ? (m_ref + __builtin_amdgcn_logf(l)) * LN2 : -FLT_MAX;
    }
}

// ---------------------------------------------------------------------------
// Split combine: one wave per (row, head); lane holds 8 of the 512 outputs.
// Math of mla_reduce (opus_attn/dsa_v32/common/mla_reduce.hpp:6-156):
// m = max lse_i, w_i = exp(lse_i - m) (0 for an empty split),
// O = sum w_i O_i / sum w_i, LSE = m + ln sum w_i (+inf when all are empty).
// grid = (rows, ceil(H / 4)), block = 256.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
dsa_mla_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_lse, int ns,
                       int rows, int H, int s_q, __bf16* __restrict__ out, int64_t o_sb, int64_t o_st,
                       int64_t o_sh, float* __restrict__ lse) {
    const int row = blockIdx.x;
    const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (head >= H) return;
    const int64_t stride = (int64_t)rows * H;
    const int64_t rh = (int64_t)row * H + head;
    float m = -FLT_MAX;
    for (int s = lane; s < ns; s += 64) m = fmaxf(m, part_lse[s * stride + rh]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    f32x4 acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    float den = 0.0f;
    for (int s = 0; s < ns; ++s) {
        const float ls = part_lse[s * stride + rh];
        const float w = ls > -FLT_MAX ? __builtin_amdgcn_exp2f((ls - m) * LOG2E) : 0.0f;
        den += w;
        const f32x4* src = reinterpret_cast<const f32x4*>(part_o + (s * stride + rh) * D_VO + 8 * lane);
        acc0 += w * src[0];
        acc1 += w * src[1];
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    const bf16x4 b0 = __builtin_convertvector(acc0 * inv, bf16x4);
    const bf16x4 b1 = __builtin_convertvector(acc1 * inv, bf16x4);
    __bf16* op = out + (int64_t)(row / s_q) * o_sb + (int64_t)(row % s_q) * o_st + (int64_t)head * o_sh + 8 * lane;
    reinterpret_cast<u32x2*>(op)[0] = __builtin_bit_cast(u32x2, b0);
    reinterpret_cast<u32x2*>(op)[1] = __builtin_bit_cast(u32x2, b1);
    if (lse && lane == 0) lse[rh] = den > 0.0f ? m + __builtin_amdgcn_logf(den) * LN2 : INFINITY;
}

// ---------------------------------------------------------------------------
// fp8 cache writer: one wave per row.  Lane l owns NoPE dims 8l..8l+7 (group
// l/16) and RoPE dim l.  Codec: e4m3fn, round to nearest even, saturating.
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned e4m3_encode(float f) {
    const unsigned bits = __float_as_uint(f);
    const unsigned sign = (bits >> 24) & 0x80u;
    const unsigned mag = bits & 0x7FFFFFFFu;
    if (mag >= 0x7F800000u) return sign | 0x7Fu;
    if (mag >= 0x43E00000u) return sign | 0x7Eu;
    const int e = (int)(mag >> 23) - 127;
    unsigned code, rest, half;
    if (e >= -6) {
        const unsigned m = mag & 0x7FFFFFu;
        code = ((unsigned)(e + 7) << 3) | (m >> 20);
        rest = m & 0xFFFFFu;
        half = 0x80000u;
    } else {
        const int sh = -6 - e;
        if (sh > 11) return sign;
        const unsigned m = (mag & 0x7FFFFFu) | 0x800000u;
        const unsigned w = 20u + (unsigned)sh;
        code = m >> w;
        rest = m & ((1u << w) - 1u);
        half = 1u << (w - 1u);
    }
    if (rest > half || (rest == half && (code & 1u))) code++;
    return sign | code;
}

__global__ void __launch_bounds__(256)
dsa_kv_quantize_kernel(const __bf16* __restrict__ src, int64_t src_stride, int64_t n_rows,
                       unsigned char* __restrict__ dst, int64_t dst_total, const int64_t* __restrict__ dst_rows) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n_rows) return;
    const int64_t dr = dst_rows ? dst_rows[r] : r;
    if (dr < 0 || dr >= dst_total) return;
    const __bf16* s = src + r * src_stride;
    float v[8];
    const u32x4 x8 = *reinterpret_cast<const u32x4*>(s + 8 * lane);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const unsigned w = x8[i >> 1];
        v[i] = __uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16));
        amax = fmaxf(amax, fabsf(v[i]));
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float scale = amax / 448.0f;
    unsigned w0 = 0, w1 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const unsigned c = scale > 0.0f ? e4m3_encode(v[i] / scale) : 0u;
        if (i < 4) w0 |= c << (8 * i); else w1 |= c << (8 * (i - 4));
    }
    unsigned char* d = dst + dr * DSA_MLA_FP8_ROW_BYTES;
    *reinterpret_cast<u32x2*>(d + 8 * lane) = u32x2{w0, w1};
    if ((lane & 15) == 0) *reinterpret_cast<float*>(d + D_NOPE + 4 * (lane >> 4)) = scale;
    reinterpret_cast<__bf16*>(d + 528)[lane] = s[D_NOPE + lane];
}

// ------------------------------------------------------------------- host

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }
int ilog2(int v) { int s = 0; while ((1 << s) < v) ++s; return s; }

int auto_splits(int64_t queries, int topk) {
    int ns = 1;
    const int min_split = (topk + MAX_CHUNK - 1) / MAX_CHUNK;
    if (queries > 0 && queries < 256) {
        const int64_t want = (256 + queries - 1) / queries;
        const int64_t by_len = (topk + 255) / 256;  // keep >= 8 tiles per split
        ns = (int)std::min<int64_t>(want, std::max<int64_t>(1, by_len));
    }
    ns = std::max(ns, min_split);
    return std::min(ns, DSA_MLA_MAX_SPLITS);
}

int validate_decode(const dsa_mla_decode_args* a, int* ns_out, int* chunk_out) {
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->B < 0 || a->s_q <= 0 || a->topk < 0) return DSA_ERR_BAD_SHAPE;
    if (a->H != HEADS) return DSA_ERR_UNSUPPORTED;
    if (a->kv_format != DSA_KV_BF16 && a->kv_format != DSA_KV_FP8_656) return DSA_ERR_BAD_FORMAT;
    if (a->kv_total_rows < 0 || a->kv_total_rows > INT32_MAX) return DSA_ERR_BAD_SHAPE;
    if (a->block_table && a->block_size <= 0) return DSA_ERR_BAD_SHAPE;
    if (a->num_splits < 0 || a->num_splits > DSA_MLA_MAX_SPLITS) return DSA_ERR_BAD_SPLITS;
    const int ns = a->num_splits ? a->num_splits : auto_splits((int64_t)a->B * a->s_q, a->topk);
    const int chunk = a->topk == 0 ? 0 : (a->topk + ns - 1) / ns;
    if (chunk > MAX_CHUNK) return a->num_splits ? DSA_ERR_BAD_SPLITS : DSA_ERR_UNSUPPORTED;
    if (a->B > 0 && a->topk > 0) {
        if (!a->q || !a->kv_cache || !a->seq_lens || !a->indices || !a->out) return DSA_ERR_NULL_POINTER;
        if ((a->q_stride_h % 8) != 0 || (a->q_stride_t % 8) != 0 || (a->q_stride_b % 8) != 0)
            return DSA_ERR_BAD_STRIDE;
        if ((a->o_stride_h % 4) != 0 || (a->o_stride_t % 4) != 0 || (a->o_stride_b % 4) != 0)
            return DSA_ERR_BAD_STRIDE;
        if (((uintptr_t)a->q & 15) || ((uintptr_t)a->kv_cache & 15) || ((uintptr_t)a->out & 7))
            return DSA_ERR_BAD_STRIDE;
    }
    if (a->B > 0 && a->topk == 0 && !a->out) return DSA_ERR_NULL_POINTER;
    *ns_out = ns;
    *chunk_out = chunk;
    return DSA_OK;
}

size_t decode_ws_bytes(const dsa_mla_decode_args* a, int ns) {
    if (ns <= 1) return 0;
    const size_t rows = (size_t)a->B * a->s_q * HEADS;
    return (size_t)ns * rows * (D_VO + 1) * sizeof(float) + 256;
}

int launch_fwd(const FwdParams& fp, int fmt, int B, int s_q, int ns, hipStream_t st) {
    dim3 grid(B, s_q, ns), block(NTHR);
    if (fmt == DSA_KV_BF16) hipLaunchKernelGGL(dsa_mla_fwd_kernel<DSA_KV_BF16>, grid, block, 0, st, fp);
    else hipLaunchKernelGGL(dsa_mla_fwd_kernel<DSA_KV_FP8_656>, grid, block, 0, st, fp);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

int launch_combine(const float* po, const float* pl, int ns, int rows, int H, int s_q, void* out, int64_t o_sb,
                   int64_t o_st, int64_t o_sh, float* lse, hipStream_t st) {
    if (rows == 0) return DSA_OK;
    dim3 grid(rows, (H + 3) / 4), block(256);
    hipLaunchKernelGGL(dsa_mla_combine_kernel, grid, block, 0, st, po, pl, ns, rows, H, s_q, (__bf16*)out, o_sb,
                       o_st, o_sh, lse);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

}  // namespace

extern "C" {

int dsa_mla_abi_version(void) { return 1; }

const char* dsa_mla_strerror(int code) {
    switch (code) {
    case DSA_OK: return "success";
    case DSA_ERR_NULL_POINTER: return "a required pointer is NULL";
    case DSA_ERR_BAD_SHAPE: return "invalid shape argument";
    case DSA_ERR_UNSUPPORTED: return "unsupported configuration (H must be 128; top-k per split <= 2048)";
    case DSA_ERR_BAD_FORMAT: return "unknown kv_format";
    case DSA_ERR_WORKSPACE: return "workspace missing or too small";
    case DSA_ERR_BAD_SPLITS: return "num_splits out of range or too small for top-k";
    case DSA_ERR_BAD_STRIDE: return "misaligned pointer or stride";
    case DSA_ERR_HIP: return "HIP runtime error";
    default: return "unknown error";
    }
}

int dsa_mla_decode_num_splits(const dsa_mla_decode_args* a, int32_t* num_splits) {
    if (!num_splits) return DSA_ERR_NULL_POINTER;
    int ns, chunk;
    const int rc = validate_decode(a, &ns, &chunk);
    if (rc) return rc;
    *num_splits = ns;
    return DSA_OK;
}

int dsa_mla_decode_workspace_size(const dsa_mla_decode_args* a, size_t* bytes) {
    if (!bytes) return DSA_ERR_NULL_POINTER;
    int ns, chunk;
    const int rc = validate_decode(a, &ns, &chunk);
    if (rc) return rc;
    *bytes = decode_ws_bytes(a, ns);
    return DSA_OK;
}

int dsa_mla_decode(const dsa_mla_decode_args* a, void* ws, size_t ws_bytes, void* stream) {
    int ns, chunk;
    const int rc = validate_decode(a, &ns, &chunk);
    if (rc) return rc;
    const size_t need = decode_ws_bytes(a, ns);
    if (need && (!ws || ws_bytes < need || ((uintptr_t)ws & 15))) return DSA_ERR_WORKSPACE;
    if (a->B == 0) return DSA_OK;
    hipStream_t st = (hipStream_t)stream;
    FwdParams fp{};
    fp.q = (const __bf16*)a->q;
    fp.q_sb = a->q_stride_b; fp.q_st = a->q_stride_t; fp.q_sh = a->q_stride_h;
    fp.kv = (const unsigned char*)a->kv_cache;
    fp.kv_total_rows = a->kv_total_rows;
    fp.kv_batch_stride = a->kv_batch_stride;
    fp.block_table = a->block_table;
    fp.bt_stride = a->block_table_stride;
    fp.block_size = a->block_table ? a->block_size : 1;
    fp.bs_shift = is_pow2(fp.block_size) ? ilog2(fp.block_size) : -1;
    fp.seq_lens = a->seq_lens;
    fp.seq_len_default = 0;
    fp.indices = a->indices;
    fp.idx_sb = a->idx_stride_b; fp.idx_st = a->idx_stride_t;
    fp.out = (__bf16*)a->out;
    fp.o_sb = a->o_stride_b; fp.o_st = a->o_stride_t; fp.o_sh = a->o_stride_h;
    fp.lse = a->lse;
    fp.B = a->B; fp.s_q = a->s_q; fp.topk = a->topk; fp.chunk = chunk;
    fp.causal = a->causal ? 1 : 0;
    fp.causal_offset = 0;
    fp.scale_log2 = a->sm_scale * LOG2E;
    if (ns > 1) {
        const size_t rows = (size_t)a->B * a->s_q * HEADS;
        fp.part_o = (float*)ws;
        fp.part_lse = (float*)((char*)ws + (size_t)ns * rows * D_VO * sizeof(float));
    }
    int r = launch_fwd(fp, a->kv_format, a->B, a->s_q, ns, st);
    if (r || ns == 1) return r;
    return launch_combine(fp.part_o, fp.part_lse, ns, a->B * a->s_q, HEADS, a->s_q, a->out, a->o_stride_b,
                          a->o_stride_t, a->o_stride_h, a->lse, st);
}

int dsa_mla_combine(const float* po, const float* pl, int32_t ns, int32_t rows, int32_t H, void* out,
                    int64_t o_sr, int64_t o_sh, float* lse, void* stream) {
    if (rows < 0 || H <= 0) return DSA_ERR_BAD_SHAPE;
    if (ns <= 0 || ns > DSA_MLA_MAX_SPLITS) return DSA_ERR_BAD_SPLITS;
    if (rows == 0) return DSA_OK;
    if (!po || !pl || !out) return DSA_ERR_NULL_POINTER;
    if (((uintptr_t)po & 15) || ((uintptr_t)out & 7) || (o_sr % 4) || (o_sh % 4)) return DSA_ERR_BAD_STRIDE;
    return launch_combine(po, pl, ns, rows, H, 1, out, o_sr, 0, o_sh, lse, (hipStream_t)stream);
}

int dsa_mla_prefill_workspace_size(const dsa_mla_prefill_args* a, size_t* bytes) {
    if (!a || !bytes) return DSA_ERR_NULL_POINTER;
    if (a->N < 0 || a->topk < 0 || a->kv_rows < 0) return DSA_ERR_BAD_SHAPE;
    if (a->H != HEADS) return DSA_ERR_UNSUPPORTED;
    if (a->topk > MAX_CHUNK) return DSA_ERR_UNSUPPORTED;
    *bytes = 0;
    return DSA_OK;
}

int dsa_mla_prefill(const dsa_mla_prefill_args* a, void* ws, size_t ws_bytes, void* stream) {
    (void)ws; (void)ws_bytes;
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->N < 0 || a->topk < 0 || a->kv_rows < 0 || a->kv_rows > INT32_MAX) return DSA_ERR_BAD_SHAPE;
    if (a->H != HEADS) return DSA_ERR_UNSUPPORTED;
    if (a->kv_format != DSA_KV_BF16 && a->kv_format != DSA_KV_FP8_656) return DSA_ERR_BAD_FORMAT;
    if (a->topk > MAX_CHUNK) return DSA_ERR_UNSUPPORTED;
    if (a->N == 0) return DSA_OK;
    if (!a->q || !a->out || (a->topk > 0 && (!a->kv || !a->indices))) return DSA_ERR_NULL_POINTER;
    if ((a->q_stride_n % 8) || (a->q_stride_h % 8) || (a->o_stride_n % 4) || (a->o_stride_h % 4))
        return DSA_ERR_BAD_STRIDE;
    if (((uintptr_t)a->q & 15) || ((uintptr_t)a->kv & 15) || ((uintptr_t)a->out & 7)) return DSA_ERR_BAD_STRIDE;
    FwdParams fp{};
    fp.q = (const __bf16*)a->q;
    fp.q_sb = a->q_stride_n; fp.q_st = 0; fp.q_sh = a->q_stride_h;
    fp.kv = (const unsigned char*)a->kv;
    fp.kv_total_rows = a->kv_rows;
    fp.kv_batch_stride = 0;
    fp.block_table = nullptr;
    fp.block_size = 1;
    fp.bs_shift = 0;
    fp.seq_lens = nullptr;
    fp.seq_len_default = a->kv_rows;
    fp.indices = a->indices;
    fp.idx_sb = a->idx_stride_n; fp.idx_st = 0;
    fp.out = (__bf16*)a->out;
    fp.o_sb = a->o_stride_n; fp.o_st = 0; fp.o_sh = a->o_stride_h;
    fp.lse = a->lse;
    fp.B = a->N; fp.s_q = 1; fp.topk = a->topk; fp.chunk = a->topk;
    fp.causal = a->causal ? 2 : 0;
    fp.causal_offset = a->causal_offset;
    fp.scale_log2 = a->sm_scale * LOG2E;
    return launch_fwd(fp, a->kv_format, a->N, 1, 1, (hipStream_t)stream);
}

int dsa_kv_quantize_fp8(const void* src, int64_t src_stride, int64_t n_rows, void* dst, int64_t dst_total,
                        const int64_t* dst_rows, void* stream) {
    if (n_rows < 0 || dst_total < 0) return DSA_ERR_BAD_SHAPE;
    if (n_rows == 0) return DSA_OK;
    if (!src || !dst) return DSA_ERR_NULL_POINTER;
    if ((src_stride % 8) || ((uintptr_t)src & 15) || ((uintptr_t)dst & 15)) return DSA_ERR_BAD_STRIDE;
    if (!dst_rows && n_rows > dst_total) return DSA_ERR_BAD_SHAPE;
    const int64_t blocks = (n_rows + 3) / 4;
    hipLaunchKernelGGL(dsa_kv_quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const __bf16*)src, src_stride, n_rows, (unsigned char*)dst, dst_total, dst_rows);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

}  // extern "C"
