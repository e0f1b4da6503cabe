// dsa_mla.hip - gfx950 (MI355X) sparse MLA decode / prefill kernels and the
// C ABI declared in include/dsa_mla.h.
//
// Forward kernel: one workgroup per (query token, top-k split).  4 waves x 32
// heads = 128 heads, so every gathered latent row is read from HBM once and
// used by all heads.  The top-k list is first resolved to physical cache rows
// and compacted (invalid entries dropped), then processed in tiles of 32 rows:
//   gather   16-byte LDS-DMA loads (global_load_lds_dwordx4) of whole rows,
//            issued 2 (bf16) / 3 (fp8) tiles ahead of use
//   dequant  fp8 rows only: cooperative conversion of the next tile into a
//            16-bit tile buffer (656-B rows: v_cvt_scalef32_pk_f16_fp8 applies
//            the power-of-two part of the per-128 scale, v_pk_mul_f16 its
//            mantissa; MXFP8 rows: exact bf16), between the PV MFMAs
//   QK^T     each wave: S^T[32 rows x its 32 heads] with 32x32x16 MFMAs (bf16,
//            or fp16 for the 656-B cache), Q held in registers
//   softmax  exp2 of the scores against a fixed per-head reference (the first
//            tile's maximum): the O accumulators are never rescaled in the loop
//   PV       each wave: O^T[its 128 dims x 128 heads] += V^T P^T, V^T read
//            with ds_read_b64_tr_b16, P exchanged between the waves in LDS
// One wave per SIMD: the wave's VALU instructions do not overlap its MFMAs, so
// the tile loops keep the non-MFMA instruction count low (one QK^T chain,
// branches rather than selects for the last-tile masks, scalar row addresses).
// bf16 caches run a software-pipelined loop (QK^T of tile t+1 and the softmax
// numerators of tile t+1 within PV of tile t, one barrier per tile).
// The structure follows the reference's one-workgroup-per-work-item decode
// (opus_attn/dsa_v32/gfx950/mla_decode_a16w16_32mxt_32nx1_template.hpp:916-1132)
// but is written from scratch for stock hipcc: no OPUS, no pinned registers,
// a top-k index form, compacted index lists and an fp16 dequant path.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "../../include/dsa_mla.h"
#include "dsa_rows.h"

namespace {

constexpr int D_QK = DSA_MLA_D_QK;
constexpr int D_NOPE = DSA_MLA_D_NOPE;
constexpr int D_VO = DSA_MLA_D_VO;
constexpr int HEADS = 128;                 // heads per workgroup (4 waves x 32)
constexpr int NWAVE = 4;
constexpr int NTHR = NWAVE * 64;
constexpr int TILE = 32;                   // latent rows per tile
constexpr int MAX_CHUNK = 2048;            // list entries a workgroup resolves at a time
// longest list (top-k, max_kv_len, max_rows): entry positions stay int32
constexpr int32_t MAX_LIST = DSA_MLA_MAX_LIST;
static_assert(MAX_LIST == INT32_MAX - MAX_CHUNK, "list positions + one chunk fit int32");
constexpr int KS_NOPE = D_NOPE / 16;       // 16-deep k-steps over the NoPE dims (32)
constexpr int KS_ALL = D_QK / 16;          // all k-steps (36)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.69314718055994531f;

constexpr int BF16_ROW = DSA_MLA_BF16_ROW_BYTES;   // 1152
constexpr int FP8_ROW = DSA_MLA_FP8_ROW_BYTES;     // 656

// Tile buffer: 32 rows of 16-bit latent values (bf16, or fp16 after dequant).
//   NoPE: row r at r * NOPE_STRIDE (1024 data bytes + 64 pad); its 16-byte
//         chunk c sits at chunk position c ^ nope_sw(r).  The pad shifts every
//         row by 4 bank groups, the XOR separates rows 4 apart, so both the K
//         fragment reads (one chunk of 16 rows) and the transposed V reads
//         (4 chunks of 4 rows) hit 16 distinct 16-byte bank groups.
//   RoPE: row r at ROPE_OFF + 128 r, chunk c (0..7) at position c ^ rope_sw(r).
constexpr int NOPE_STRIDE = 1088;
constexpr int ROPE_OFF = TILE * NOPE_STRIDE;         // 34816
constexpr int TILE_BYTES = ROPE_OFF + TILE * 128;    // 38912
constexpr int RAW_BYTES = TILE * FP8_ROW;            // raw fp8 tile, rows back to back (20992)
constexpr int FP8_CHUNKS = RAW_BYTES / 16;           // 16-byte chunks of a raw tile (1312)
constexpr int FP8_LOADS = (FP8_CHUNKS + 63) / 64;    // wave-wide loads per raw tile (21)
constexpr int RAW_STRIDE = FP8_LOADS * 1024;         // raw slot padded to whole loads (21504)
constexpr int FP8_LPW = (FP8_LOADS + NWAVE - 1) / NWAVE;  // loads of wave 0 (6); the others 5
constexpr int BF16_LPW = TILE / NWAVE + 1;           // 8 NoPE rows + one 8-row RoPE block
constexpr int FP8_SCALE_OFF = D_NOPE;                // 4 fp32 scales
constexpr int FP8_ROPE_OFF = D_NOPE + 16;            // 64 bf16 RoPE values
// MXFP8 raw slot, one region per stream (every DMA load reads one stream):
// NoPE codes of row r at 512 r (loads 0..15, two rows each), RoPE at
// MX_ROPE_OFF + 128 r (loads 16..19, eight rows each), the 16 E8M0 scales at
// MX_SC_OFF + 16 r (load 20; its upper 32 lanes repeat rows 0..31 into the
// slot's padding).  Same 21 loads per tile as the 656-B rows.  In the V3.2
// format the 16-byte pieces of a row are permuted: NoPE piece c of row r at
// position c ^ (r & 15), RoPE piece c at c ^ (r & 7), so that the QK^T reads
// of one piece over 16 rows hit distinct bank groups.
constexpr int MX_ROPE_OFF = TILE * D_NOPE;            // 16384
constexpr int MX_SC_OFF = MX_ROPE_OFF + TILE * 128;   // 20480
static_assert(MX_SC_OFF + 1024 <= 21 * 1024, "MXFP8 raw slot fits the 656-B slot");

__device__ __forceinline__ int nope_sw(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int rope_sw(int r) { return (r >> 1) & 7; }

// LDS layout per cache format: tile buffers 0 and 1, then a ring region
// (bf16: the third tile buffer; fp8: three raw slots), then the row list.
template <int FMT>
struct Lay {
    // 656-B rows: fp16 MFMA operands (the per-128 fp32 scale's mantissa is
    // applied in fp16, so the dequantised values are fp16, not bf16)
    static constexpr bool F16 = FMT == DSA_KV_FP8_656;
    // MXFP8 split streams (E8M0 scales, dequantised exactly to bf16): the
    // V3.2 decode format, or the V4 format (448 fp8 NoPE values whose 14
    // scales follow them in the same 512-byte stream row, then 64 bf16 RoPE)
    static constexpr bool MX = FMT == DSA_KV_MXFP8 || FMT == DSA_KV_MXFP8_V4;
    static constexpr bool V4MX = FMT == DSA_KV_MXFP8_V4;
    // MXFP8 split streams (V3.2): the NoPE part of QK^T runs as scaled fp8
    // MFMAs straight from the raw slot (Q and K both carry E8M0 blocks of 32)
    static constexpr bool SQK = FMT == DSA_KV_MXFP8;
    // fp8 caches (any): raw-tile ring, dequant stage into the tile buffers
    static constexpr bool FP8 = F16 || MX;
    // 512-value rows: K = V = the whole row (V4 prefill)
    static constexpr bool D512 = FMT == DSA_KV_BF16_D512 || FMT == DSA_KV_MXFP8_V4;
    // LDS-DMA loads per raw tile: V4 rows need no separate scale load
    static constexpr int LOADS = V4MX ? 20 : FP8_LOADS;
    // k-steps of QK^T whose Q values come from the fp8 NoPE stream
    static constexpr int Q8_KS = V4MX ? DSA_MLA_V4_NOPE / 16 : KS_NOPE;
    static constexpr int RING_BYTES = FP8 ? 3 * RAW_STRIDE : TILE_BYTES;
    static constexpr int LPW = FP8 ? FP8_LPW : (D512 ? TILE / NWAVE : BF16_LPW);  // max DMA loads per wave per tile
    static constexpr int KS = D512 ? KS_NOPE : KS_ALL;    // 16-deep k-steps of QK^T
    // p = exp2(s - m_ref) may grow to 2^TAU over the reference before a
    // restart: fp16 P (656-B cache) is finite below 2^16, bf16 P below 2^128.
    static constexpr float TAU = F16 ? 15.0f : 100.0f;
};

#include "dsa_lds.h"

// Wait states between the O MFMAs (inline asm) and VALU accesses of O: 24
// covers a VALU read or write after the last 8-pass MFMA and an MFMA after a
// VALU write.  Every O tile is an in/out operand, so no access of O moves
// across it.
__device__ __forceinline__ void o_fence(f32x16 (&o)[16]) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+a"(o[0]), "+a"(o[1]), "+a"(o[2]), "+a"(o[3]), "+a"(o[4]), "+a"(o[5]),
                   "+a"(o[6]), "+a"(o[7]), "+a"(o[8]), "+a"(o[9]), "+a"(o[10]), "+a"(o[11]),
                   "+a"(o[12]), "+a"(o[13]), "+a"(o[14]), "+a"(o[15]));
}

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
    const int32_t* kv_indptr;    // CSR form (NULL: top-k form): rows kv_indices[kv_indptr[b] + k]
    const int32_t* kv_indices;
    // V4 prefill form (ind_pre != NULL): query b attends idx_pre[ind_pre[b] ..
    // ind_pre[b+1]) of kv, then idx_ext[ind_ext[b] .. ind_ext[b+1]) of kv2
    const int32_t* ind_pre;
    const int32_t* idx_pre;
    const int32_t* ind_ext;
    const int32_t* idx_ext;
    const unsigned char* kv2;    // second row pool (V4 extend rows)
    int64_t kv2_rows;
    int64_t row_bytes;           // bytes between cache rows (bf16, 656-B and 512-value rows)
    const float* attn_sink;      // per-head sink in the softmax denominator, or NULL
    // MXFP8 split streams: q carries the bf16 RoPE part of Q, kv the fp8 NoPE
    // codes; strides of the fp8 / E8M0 streams in bytes
    const unsigned char* q8;     // fp8 NoPE part of Q
    int64_t q8_sb, q8_st, q8_sh;
    const unsigned char* qsc;    // E8M0 scales of Q (16 per head)
    int64_t qsc_sb, qsc_st, qsc_sh;
    const unsigned char* kv_sc;  // E8M0 scales of the cache rows
    const unsigned char* kv_ro;  // bf16 RoPE of the cache rows
    const unsigned char* kv2_ro; // bf16 RoPE of the second pool's rows (V4 fp8)
    uint32_t kvn_st, kvs_st, kvr_st;   // row strides of kv / kv_sc / kv_ro (bytes)
    __bf16* out;
    int64_t o_sb, o_st, o_sh;
    float* lse;
    float* part_o;               // [splits][B*s_q][H][512] fp32, NULL when unsplit
    float* part_lse;             // [splits][B*s_q][H]
    int32_t B, s_q, topk, chunk;
    int32_t H;                   // heads of a query token (any H >= 1)
    int32_t hgroups;             // workgroups per (query token, split): ceil(H / 128)
    // CSR work plan (NULL: one workgroup per (query token, split)): item i =
    // (query row b * s_q + t, first entry, end entry, partial slot or -1 for a
    // token the plan left whole); plan_hdr[0] = number of items
    const int4* plan_items;
    const int32_t* plan_hdr;
    int32_t causal;              // 1: decode rule  j <= L - s_q + t
                                 // 2: prefill rule j <= b + causal_offset
    int64_t causal_offset;
    int32_t reverse;             // 1: workgroup x takes query token B-1-x (prefill)
    float scale_log2;            // sm_scale * log2(e)
};

// CSR work-plan item field w: bits 0..29 hold the partial slot + 1 (0: the
// item writes its row's output directly), bit 30 marks the row's last item.
constexpr int PLAN_LAST = 1 << 30;
__host__ __device__ inline int plan_item_w(int slot, bool last) { return (slot + 1) | (last ? PLAN_LAST : 0); }
__host__ __device__ inline int plan_item_slot(int w) { return (w & (PLAN_LAST - 1)) - 1; }
// plan header: [0] items, [1] split rows, [2] chunk, then the B, s_q and
// max_kv_len it was built for
constexpr int PLAN_HDR_B = 3, PLAN_HDR_SQ = 4, PLAN_HDR_MAXLEN = 5;

// A global-memory pointer from its address (a generic pointer of unknown
// origin would be accessed with flat loads).
template <class T>
__device__ __forceinline__ T* gptr(uintptr_t u) {
    return (T*)(__attribute__((address_space(1))) T*)u;
}

// A wave-uniform int32 read through the scalar cache (the constant address
// space: an s_load, counted apart from the vector loads, so that waiting for it
// does not wait for vector loads issued earlier).  For data the kernel
// reading it never writes (the call's index arrays and lengths).
__device__ __forceinline__ int32_t sload(const int32_t* ptr) {
    return *(const __attribute__((address_space(4))) int32_t*)(uintptr_t)ptr;
}

// Inclusive prefix sum over the wave's lanes of v (0 <= v < 16): from the
// ballots of v's four bits, each counted below the lane (v_mbcnt), with no
// LDS round trip.
__device__ __forceinline__ int wave_incl_sum16(int v) {
    int excl = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint64_t m = __builtin_amdgcn_ballot_w64(((v >> k) & 1) != 0);
        excl += (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u)) << k;
    }
    return excl + v;
}

// Physical cache rows of top-k entries jv of query b (-1 where skipped), in
// two stages so that a caller can issue other loads between them.
// topk_ents: paged, the block-table entry of each entry's block (-1 for a
// skipped entry; a negative table entry is skipped as well, its rows are
// below 0), all N reads issued before any is waited for (one memory round
// trip, not N); flat, the entry's block index (-1: skipped).
template <int N>
__device__ __forceinline__ void topk_ents(const FwdParams& p, int b, int64_t jmax, const int32_t (&jv)[N],
                                          int32_t (&ent)[N]) {
    if (p.block_table) {
        const int32_t* bt = p.block_table + (int64_t)b * p.bt_stride;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const int32_t blk = dsa_rows::topk_block(jv[e], jmax, p.block_size, p.bs_shift);
            ent[e] = blk >= 0 ? bt[blk] : -1;
        }
    } else {
#pragma unroll
        for (int e = 0; e < N; ++e) ent[e] = dsa_rows::topk_block(jv[e], jmax, p.block_size, p.bs_shift);
    }
}
// topk_rows_of: the rows, from the entries and what topk_ents gave for them
template <int N>
__device__ __forceinline__ void topk_rows_of(const FwdParams& p, int b, const int32_t (&jv)[N],
                                             const int32_t (&ent)[N], int32_t (&rows)[N]) {
    const int64_t flat = (int64_t)b * p.kv_batch_stride;
    const bool paged = p.block_table != nullptr;
#pragma unroll
    for (int e = 0; e < N; ++e)
        rows[e] = ent[e] < 0 ? -1
                             : (int32_t)dsa_rows::topk_finish(jv[e], 0, paged ? ent[e] : 0, paged, p.block_size,
                                                              p.bs_shift, flat, p.kv_total_rows);
}
template <int N>
__device__ __forceinline__ void topk_rows(const FwdParams& p, int b, int64_t jmax, const int32_t (&jv)[N],
                                          int32_t (&rows)[N]) {
    int32_t ent[N];
    topk_ents(p, b, jmax, jv, ent);
    topk_rows_of(p, b, jv, ent, rows);
}

// One piece of the fp8 dequant in flight: codes + scale, or 16 RoPE bytes.
struct DeqPiece {
    u32x4 v;
};
constexpr int DEQ_PIECES = TILE / NWAVE + 1;

// fp8 e4m3 x e4m3, 32x32x64, with E8M0 block scales: byte `sel` of sa / sb
// (a constant once the caller's loop is unrolled)
typedef int i32x8 __attribute__((ext_vector_type(8)));
template <int SEL>
__device__ __forceinline__ f32x16 mfma_scale8_sel(i32x8 a, i32x8 b, f32x16 c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, SEL, sa, SEL, sb);
}
__device__ __forceinline__ f32x16 mfma_scale8(int sel, i32x8 a, i32x8 b, f32x16 c, int sa, int sb) {
    switch (sel) {
        case 0: return mfma_scale8_sel<0>(a, b, c, sa, sb);
        case 1: return mfma_scale8_sel<1>(a, b, c, sa, sb);
        case 2: return mfma_scale8_sel<2>(a, b, c, sa, sb);
        default: return mfma_scale8_sel<3>(a, b, c, sa, sb);
    }
}

__device__ __forceinline__ f32x16 mfma_bf16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_f16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// O += A B on an AGPR accumulator.  Inline asm, so the O accumulators are
// bound to AGPRs for the whole kernel while every other MFMA (QK^T) keeps its
// accumulator in VGPRs: the AGPR file is exactly the 16 O tiles, and an
// accumulator of the compiler's choosing there would displace one of them.
// The compiler does not see these as MFMAs, so the wait states it would add
// are written out: "s_nop 1" covers a VALU write of an operand just before
// (2 wait states); o_fence() covers VALU accesses of O around the loop.
template <bool F16>
__device__ __forceinline__ void mfma_o(f32x16& acc, u32x4 a, u32x4 b) {
    if constexpr (F16)
        asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
    else
        asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// bf16 pair times s (a power of two) -> fp16 pair.  Exact for |x s| in
// [2^-14, 65504]; smaller values go to fp16 subnormals (truncated, absolute
// error < 2^-24).  s = 1 leaves every value as it is.
__device__ __forceinline__ unsigned bf16x2_to_f16x2(unsigned w, float s) {
    const float lo = __uint_as_float(w << 16) * s, hi = __uint_as_float(w & 0xFFFF0000u) * s;
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}
// bf16 pair times s (a power of two) -> bf16 pair: exact unless a product
// leaves bf16's normal range (|x s| < 2^-126).
__device__ __forceinline__ unsigned bf16x2_scale(unsigned w, float s) {
    const f32x2 v = {__uint_as_float(w << 16) * s, __uint_as_float(w & 0xFFFF0000u) * s};
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
}
// fp16 range of the 656-B path.  Its K / V values are fp16(code * 2^e) *
// fp16(mantissa) with scale = mantissa * 2^e, so every value of a row stays
// below 448 * 128 = 57344 < 65504 when the row's scales are below 128.  A
// scale of 128 or more, a negative or non-finite one (fp32 bits, unsigned,
// >= those of 128.0) is outside the path's range: the query token's outputs
// are then NaN, never a silently wrong attention.
constexpr unsigned FP8_SCALE_LIMIT_BITS = 0x43000000u;   // 128.0f

// 8 fp8 e4m3 codes (two dwords, low byte first) times 2^(e - 127) -> 8 bf16.
// Exact: the scale is a power of two and bf16 has fp32's exponent range, so
// every product is a bf16 value.  The scale operand is the fp32 2^(e - 127)
// (its exponent field is e); v_cvt_scalef32_pk_bf16_fp8 applies it.
__device__ __forceinline__ u32x4 mx_to_bf16(unsigned c0, unsigned c1, unsigned e) {
    const float sf = __uint_as_float(e << 23);
    return u32x4{__builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)c0, sf, false)),
                 __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)c0, sf, true)),
                 __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)c1, sf, false)),
                 __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)c1, sf, true))};
}

// The attention sink joins the softmax denominator as exp(sink), with the
// maximum taken over the scores and the sink together (mla_v4_host.cc:469-472).
// In log2 units: the rows' sum l_rows is taken against reference m; the result
// is the denominator l_out against reference m_out = max(m, sink2), so a sink
// far above every score (or far below) neither overflows nor underflows the
// sum.  O then scales by 2^(m - m_out) / l_out, and LSE = m_out + log2 l_out.
__device__ __forceinline__ void add_sink(float l_rows, float m, float sink2, float& l_out, float& m_out) {
    const float d = sink2 - m;
    if (d > 0.0f) {
        l_out = __builtin_fmaf(l_rows, __builtin_amdgcn_exp2f(-d), 1.0f);
        m_out = sink2;
    } else {
        l_out = l_rows + __builtin_amdgcn_exp2f(d);
        m_out = m;
    }
}

// ---------------------------------------------------------------------------
// Fused sparse-MLA forward: one workgroup per (query token, split).
// grid = (B, s_q, num_splits), block = 256.
// ---------------------------------------------------------------------------
template <int FMT>
__global__ void __launch_bounds__(NTHR) __attribute__((amdgpu_waves_per_eu(1, 1)))
dsa_mla_fwd_kernel(const FwdParams p) {
    using L = Lay<FMT>;
    constexpr bool FP8 = L::FP8;
    // Separate LDS objects for the tile buffers: the compiler can then prove
    // that the dequant stores into one buffer never alias the K / V reads of
    // the other, and interleave them with the MFMAs.
    __shared__ __attribute__((aligned(1024))) unsigned char s_tile0[TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) unsigned char s_tile1[TILE_BYTES];
    // bf16: the third ring buffer; fp8: the three raw slots
    __shared__ __attribute__((aligned(1024))) unsigned char s_ring[L::RING_BYTES];
    __shared__ int32_t s_rows_arr[MAX_CHUNK];
    // P exchange: [u][source wave][hi][head lane] x 16 bytes (8 P values), so
    // a B-operand fragment of the PV MFMA is one contiguous 16-byte read.
    // bf16 caches keep two (the P of tile it+1 is written while tile it's is read).
    constexpr int PXB = 2 * NWAVE * 64 * 16;
    __shared__ __attribute__((aligned(16))) unsigned char s_p[(FP8 ? 1 : 2) * PXB];
    __shared__ int s_misc_arr[16];            // [0..3] wave sums, [4] restart flag
    const lds_ptr T0 = (lds_ptr)s_tile0;
    const lds_ptr T1 = (lds_ptr)s_tile1;
    const lds_ptr RING = (lds_ptr)s_ring;
    const lds_ptr PX = (lds_ptr)s_p;
    LDS_AS int32_t* const s_rows = (LDS_AS int32_t*)s_rows_arr;
    LDS_AS int* const s_misc = (LDS_AS int*)s_misc_arr;

    // Every argument the prologue reads, of every form, loaded in one batch:
    // an asm statement that takes them as inputs must have them all, so their
    // scalar loads go out together.  Left to the compiler, each branch below
    // loaded its fields where it first used them, a chain of about nine
    // memory round trips before the first list entry was requested.  (Inputs
    // only, but for Q's address, which the compiler otherwise reloaded in a
    // round trip of its own just before the Q loads.)
    const __bf16* q_base = p.q;
    int64_t q_sb = p.q_sb, q_st = p.q_st, q_sh = p.q_sh;
    asm volatile("" : "+s"(q_base), "+s"(q_sb), "+s"(q_st), "+s"(q_sh)
                 : "s"(gridDim.x), "s"(gridDim.z), "s"(p.kv_total_rows),
                 "s"(p.kv_batch_stride), "s"(p.block_table), "s"(p.bt_stride), "s"(p.block_size),
                 "s"(p.bs_shift), "s"(p.seq_lens), "s"(p.seq_len_default), "s"(p.indices), "s"(p.idx_sb),
                 "s"(p.idx_st), "s"(p.kv_indptr), "s"(p.kv_indices), "s"(p.ind_pre), "s"(p.idx_pre),
                 "s"(p.ind_ext), "s"(p.idx_ext), "s"(p.kv2_rows), "s"(p.B), "s"(p.s_q), "s"(p.topk),
                 "s"(p.chunk), "s"(p.H), "s"(p.hgroups), "s"(p.plan_items), "s"(p.plan_hdr), "s"(p.causal),
                 "s"(p.causal_offset), "s"(p.reverse));
    if constexpr (Lay<FMT>::MX)
        asm volatile("" ::"s"(p.q8), "s"(p.q8_sb), "s"(p.q8_st), "s"(p.q8_sh), "s"(p.qsc), "s"(p.qsc_sb),
                     "s"(p.qsc_st), "s"(p.qsc_sh));

    // blockIdx.x = work item * hgroups + head group.  A work item is query
    // token b = blockIdx.x, t = blockIdx.y, split blockIdx.z of its list; or,
    // under a CSR plan, an entry of the plan's item table.
    const int gx = p.hgroups == 1 ? (int)blockIdx.x : (int)blockIdx.x / p.hgroups;
    const int hbase = p.hgroups == 1 ? 0 : HEADS * ((int)blockIdx.x % p.hgroups);
    // Prefill runs its tokens last to first: later tokens see more rows, and
    // with the longest lists dispatched first the CUs finish together instead
    // of idling behind the last long workgroups.
    int b = p.reverse ? (int)(gridDim.x / p.hgroups) - 1 - gx : gx, t = blockIdx.y;
    const int split = blockIdx.z;
    int item_k0 = 0, item_k1 = 0, item_slot = -1;
    bool item_last = false;
    if (p.plan_items) {
        // The plan must be the one built for this call's kv_indptr, B, s_q
        // and max_kv_len.  A plan built for other arguments lays out other
        // items and partial slots: then every query row's outputs are NaN,
        // and nothing else is read or written.
        // (the header's fields are read together, then compared: one round trip)
        const int32_t hdr_items = sload(p.plan_hdr), hdr_b = sload(p.plan_hdr + PLAN_HDR_B),
                      hdr_sq = sload(p.plan_hdr + PLAN_HDR_SQ), hdr_len = sload(p.plan_hdr + PLAN_HDR_MAXLEN);
        if ((hdr_b != p.B) | (hdr_sq != p.s_q) | (hdr_len != p.chunk)) {
            // (the grid holds at least B * s_q workgroups per head group)
            if (gx < p.B * p.s_q) {
                const int bq = gx / p.s_q, tq = gx - bq * p.s_q;
                __bf16* const orow = p.out + (int64_t)bq * p.o_sb + (int64_t)tq * p.o_st;
                const unsigned nan2 = 0x7FC07FC0u;    // two bf16 NaNs
                for (int i = (int)threadIdx.x; i < HEADS * (D_VO / 4); i += NTHR) {
                    const int hh = hbase + i / (D_VO / 4);
                    if (hh < p.H)
                        reinterpret_cast<u32x2*>(orow + (int64_t)hh * p.o_sh)[i % (D_VO / 4)] = u32x2{nan2, nan2};
                }
                for (int hh = (int)threadIdx.x; hh < HEADS; hh += NTHR)
                    if (p.lse && hbase + hh < p.H) p.lse[(int64_t)gx * p.H + hbase + hh] = __builtin_nanf("");
            }
            return;
        }
        // Items are in row order, so the s_q rows of a batch (MTP tokens with
        // one list) are consecutive items.  Workgroups go to the 8 XCDs in
        // turn: within each group of 8 s_q workgroups, item s_q c + u runs on
        // XCD c, so a batch's tokens share that XCD's L2 and its rows are
        // fetched from HBM once.  (The grid is a multiple of 8 s_q.)
        int item = gx;
        if (p.hgroups == 1) {
            const int G = 8 * p.s_q, j = gx / G, rem = gx - j * G;
            item = G * j + p.s_q * (rem & 7) + (rem >> 3);
        }
        // the grid covers the most items a plan can hold: past the plan's
        // count the whole workgroup leaves before any barrier
        if (item >= hdr_items) return;
        const int4 w = p.plan_items[item];
        const int qrow_i = __builtin_amdgcn_readfirstlane(w.x);
        if ((unsigned)qrow_i >= (unsigned)(p.B * p.s_q)) return;
        b = qrow_i / p.s_q;
        t = qrow_i - b * p.s_q;
        item_k0 = __builtin_amdgcn_readfirstlane(w.y);
        item_k1 = __builtin_amdgcn_readfirstlane(w.z);
        const int ww = __builtin_amdgcn_readfirstlane(w.w);
        item_slot = plan_item_slot(ww);
        item_last = (ww & PLAN_LAST) != 0;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5, r32 = lane & 31;
    const int head = wave * 32 + r32;         // head within the group (LDS exchanges)
    // The query's head: heads past H (H not a multiple of 128) are computed on
    // a copy of head H-1 and never stored.
    const int head_g = hbase + head;
    const int head_q = min(head_g, p.H - 1);
    if (tid == 0) {
        s_misc[4] = 0;    // restart flag
        s_misc[5] = 0;    // 656-B rows: a scale outside the fp16 path's range was read
    }

    // ---- 0. Q fragments (B operand of S^T = K Q^T): lane -> head r32, k-chunk hi ----
    // Loaded by load_q() once the first index loads are out (section 1): the
    // loads return in order, so entries and block-table reads issued after Q
    // would wait for all of Q as well.
    u32x4 qf[L::KS];
    u32x4 q_scales = {0, 0, 0, 0};   // MXFP8: the 16 E8M0 scales of this head's Q
    unsigned q_sc8[2] = {0u, 0u};    // scaled QK^T: the E8M0 bytes of blocks 2 k8 + hi (k8 = 4 i + byte)
    auto load_q = [&]() {
        if constexpr (L::SQK) {
            // B operand of the scaled fp8 MFMA (64-deep k-steps k8): lane (head,
            // hi) holds codes 64 k8 + 16 hi .. +15 and 64 k8 + 32 + 16 hi .. +15,
            // in qf[2 k8] and qf[2 k8 + 1]; RoPE as bf16 in qf[KS_NOPE ..]
            // (the lane offset from a fresh copy of the lane id: shared with the
            // epilogue's, it stayed live across the tile loop and spilled)
            const unsigned char* q8p = p.q8 + (int64_t)b * p.q8_sb + (int64_t)t * p.q8_st + (int64_t)head_q * p.q8_sh +
                                       16 * (opaque_here(lane) >> 5);
#pragma unroll
            for (int k8 = 0; k8 < KS_NOPE / 4; ++k8) {
                qf[2 * k8] = *reinterpret_cast<const u32x4*>(q8p + 64 * k8);
                qf[2 * k8 + 1] = *reinterpret_cast<const u32x4*>(q8p + 64 * k8 + 32);
            }
            q_scales = *reinterpret_cast<const u32x4*>(p.qsc + (int64_t)b * p.qsc_sb + (int64_t)t * p.qsc_st +
                                                       (int64_t)head_q * p.qsc_sh);
            const __bf16* qp = gptr<const __bf16>((uintptr_t)q_base) + (int64_t)b * q_sb + (int64_t)t * q_st +
                                (int64_t)head_q * q_sh + 8 * hi;
#pragma unroll
            for (int ks = KS_NOPE; ks < L::KS; ++ks)
                qf[ks] = *reinterpret_cast<const u32x4*>(qp + 16 * (ks - KS_NOPE));
        } else if constexpr (L::MX) {
            // fp8 codes of dims 16ks + 8hi .. +7 in the low half of qf[ks],
            // converted to bf16 once they have landed; RoPE as bf16
            const unsigned char* q8p = p.q8 + (int64_t)b * p.q8_sb + (int64_t)t * p.q8_st + (int64_t)head_q * p.q8_sh + 8 * hi;
#pragma unroll
            for (int ks = 0; ks < L::Q8_KS; ++ks) {
                const u32x2 c = *reinterpret_cast<const u32x2*>(q8p + 16 * ks);
                qf[ks] = u32x4{c[0], c[1], 0u, 0u};
            }
            q_scales = *reinterpret_cast<const u32x4*>(p.qsc + (int64_t)b * p.qsc_sb + (int64_t)t * p.qsc_st +
                                                       (int64_t)head_q * p.qsc_sh);
            const __bf16* qp = gptr<const __bf16>((uintptr_t)q_base) + (int64_t)b * q_sb + (int64_t)t * q_st +
                                (int64_t)head_q * q_sh + 8 * hi;
#pragma unroll
            for (int ks = L::Q8_KS; ks < L::KS; ++ks)
                qf[ks] = *reinterpret_cast<const u32x4*>(qp + 16 * (ks - L::Q8_KS));
        } else {
            const __bf16* qp = gptr<const __bf16>((uintptr_t)q_base) + (int64_t)b * q_sb + (int64_t)t * q_st +
                                (int64_t)head_q * q_sh + 8 * hi;
#pragma unroll
            for (int ks = 0; ks < L::KS; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qp + 16 * ks);
        }
    };

    // ---- 1. resolve this split's index chunk into a compacted row list ----
    // Top-k form: logical positions through the block table, bounded by
    // seq_len and the causal rule.  CSR form: physical rows
    // kv_indices[kv_indptr[b] + k] for k < kv_indptr[b+1] - kv_indptr[b] -
    // (s_q - 1 - t), the reference's count-based MTP causality
    // (opus_attn/dsa_v32/common/host.cc:524-526); a row outside the cache is
    // skipped.
    int k0 = p.plan_items ? item_k0 : split * p.chunk;
    int k1;
    int64_t jmax = 0;
    const int32_t* idx;
    int64_t v4_np = 0, v4_eb = 0;
    // the splits of a query cover gridDim.z * chunk entries of its list
    const int64_t k_cap = (int64_t)gridDim.z * p.chunk;
    bool truncated = false;
    if (L::D512 && p.ind_pre) {
        // V4: prefix rows of kv, then extend rows of kv2 (tagged with POOL2);
        // a decreasing indptr pair counts as an empty range
        const int64_t pb = sload(p.ind_pre + b);
        v4_np = max((int64_t)sload(p.ind_pre + b + 1) - pb, (int64_t)0);
        v4_eb = sload(p.ind_ext + b);
        const int64_t ne = max((int64_t)sload(p.ind_ext + b + 1) - v4_eb, (int64_t)0);
        // the token's list (at most max_rows = p.topk entries: a longer one is
        // cut, NaN) split into gridDim.z parts of whole tiles, as the
        // reference's split-K prefill cuts prefix-then-extend rows
        // (opus_attn/dsa_v4/common/mla_prefill_split.h:34-44)
        const int64_t n_b = min(v4_np + ne, (int64_t)p.topk);
        truncated = v4_np + ne > p.topk;
        const int64_t per = (n_b + gridDim.z - 1) / gridDim.z;
        const int64_t cb = (per + TILE - 1) / TILE * TILE;
        k0 = (int)min((int64_t)split * cb, n_b);
        k1 = (int)min((int64_t)k0 + cb, n_b);
        idx = p.idx_pre + pb;
    } else if (p.kv_indptr) {
        const int64_t kb = sload(p.kv_indptr + b);
        const int64_t count = (int64_t)sload(p.kv_indptr + b + 1) - kb - (p.s_q - 1 - t);
        k1 = (int)min(p.plan_items ? (int64_t)item_k1 : (int64_t)k0 + p.chunk, count);
        truncated = count > k_cap;
        // a row's last item ends at the length the plan was built for: a list
        // that has changed since is flagged (NaN), not silently cut
        if (item_last && (int64_t)item_k1 != max(count, (int64_t)0)) truncated = true;
        idx = p.kv_indices + kb;
    } else {
        k1 = (int)min((int64_t)k0 + p.chunk, (int64_t)p.topk);
        idx = p.indices + (int64_t)b * p.idx_sb + (int64_t)t * p.idx_st;
    }
    // The split's entries are taken MAX_CHUNK at a time (the row list holds
    // one chunk); the softmax state and the O accumulators carry over from
    // one chunk to the next, so a list of any length needs no partials.  An
    // empty range is one empty chunk.
    const int nchunks = k1 > k0 ? (k1 - k0 + MAX_CHUNK - 1) / MAX_CHUNK : 1;

    constexpr int PER_T = MAX_CHUNK / NTHR;  // 8 entries per thread and chunk
    // the entries of chunk c (-1 past the split's end), all loads issued
    // before any is used; a V4 entry k is an extend entry from k = v4_np on
    auto load_entries = [&](int c, int32_t (&jv)[PER_T]) {
        const int kc0 = k0 + c * MAX_CHUNK;
        const int kc1 = min(kc0 + MAX_CHUNK, k1);
#pragma unroll
        for (int e = 0; e < PER_T; ++e) {
            const int k = kc0 + tid * PER_T + e;
            if (k >= kc1) jv[e] = -1;
            else jv[e] = L::D512 && p.ind_pre && k >= v4_np ? p.idx_ext[v4_eb + (k - v4_np)] : idx[k];
        }
    };
    // Chunk 0's entries go out before Q, and a paged top-k list's block-table
    // reads for them as well (both are waited for before the rows are formed,
    // which then does not wait for Q); a flat list's rows need no second read.
    // The first tiles' gathers are then issued while Q is still in flight.
    int32_t jv0[PER_T], ent0[PER_T];
    load_entries(0, jv0);
    const bool topk_form = !(L::D512 && p.ind_pre) && !p.kv_indptr;
    if (topk_form) {
        // the bound on positions, from seq_len and the causal rule (a scalar
        // load, in flight with the entries)
        const int64_t Lq = p.seq_lens ? (int64_t)sload(p.seq_lens + b) : p.seq_len_default;
        jmax = Lq;
        if (p.causal == 1) jmax = min(Lq, Lq - p.s_q + t + 1);
        else if (p.causal == 2) jmax = min(Lq, (int64_t)b + p.causal_offset + 1);
    }
    const bool topk_paged = topk_form && p.block_table;
    if (topk_paged) topk_ents(p, b, jmax, jv0, ent0);
    load_q();

    // entries [kc0, min(kc0 + MAX_CHUNK, k1)) -> the compacted row list;
    // sets n_valid and ntiles (ends with a workgroup barrier).  preloaded:
    // chunk 0 from jv0 / ent0.
    int n_valid = 0, ntiles = 0;
    bool any_rows = false;
    auto resolve_chunk = [&](int c, bool preloaded) {
        const int kc0 = k0 + c * MAX_CHUNK;
        int32_t rows_local[PER_T];
        int cnt = 0;
        {
            // the rules of dsa_rows.h; a V4 entry is checked against the pool
            // its list names
            int32_t jv[PER_T];
            if (preloaded) {
#pragma unroll
                for (int e = 0; e < PER_T; ++e) jv[e] = jv0[e];
            } else {
                load_entries(c, jv);
            }
            if (L::D512 && p.ind_pre) {
#pragma unroll
                for (int e = 0; e < PER_T; ++e)
                    rows_local[e] = kc0 + tid * PER_T + e >= v4_np ? dsa_rows::v4_extend_row(jv[e], p.kv2_rows)
                                                                   : dsa_rows::v4_prefix_row(jv[e], p.kv_total_rows);
            } else if (p.kv_indptr) {
#pragma unroll
                for (int e = 0; e < PER_T; ++e) rows_local[e] = dsa_rows::csr_row(jv[e], p.kv_total_rows);
            } else {
                int32_t ent[PER_T];
                if (preloaded && topk_paged) {
#pragma unroll
                    for (int e = 0; e < PER_T; ++e) ent[e] = ent0[e];
                } else {
                    topk_ents(p, b, jmax, jv, ent);
                }
                topk_rows_of(p, b, jv, ent, rows_local);
            }
#pragma unroll
            for (int e = 0; e < PER_T; ++e) cnt += rows_local[e] >= 0 ? 1 : 0;
        }
        const int incl = wave_incl_sum16(cnt);
        // (the barrier also ends every wave's use of the previous chunk's
        // row list, tile buffers and P buffers)
        if (lane == 63) s_misc[wave] = incl;
        __syncthreads();
        int wbase = 0, nv = 0;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) {
            const int s = s_misc[w];
            wbase += w < wave ? s : 0;
            nv += s;
        }
        {
            int pos = wbase + incl - cnt;
#pragma unroll
            for (int e = 0; e < PER_T; ++e)
                if (rows_local[e] >= 0) s_rows[pos++] = rows_local[e];
        }
        n_valid = nv;
        ntiles = (nv + TILE - 1) / TILE;
        any_rows = any_rows || nv > 0;
        __syncthreads();
        // Pad the last tile with copies of the first valid row: every gathered
        // row is finite cache data, and the softmax masks the padding rows.
        if (tid < TILE && nv > 0 && nv + tid < ntiles * TILE) s_rows[nv + tid] = s_rows[0];
        __syncthreads();
    };

    // bf16 ring slot -> tile buffer
    auto slot_buf = [&](int s) -> lds_ptr { return s == 0 ? T0 : (s == 1 ? T1 : RING); };

    // ---- 2. gather: rows of tile `ti` -> ring slot `slot` ----
    // Every load is a full wave-wide LDS-DMA load of 1 KB: the number of
    // loads a CU can keep in flight is limited, so each one carries as much
    // as it can.  bf16: wave w loads NoPE rows 8w..8w+7 (one row per load)
    // plus one load covering the 8 RoPE blocks; fp8: the raw tile's 1312
    // 16-byte chunks (rows back to back) are 21 loads, wave w taking loads
    // w, w+4, ... (6 for wave 0, 5 for the others).  The row ids of the next
    // tile to issue are read from the row list a step ahead (GatherRows).
    struct GatherRows {
        int32_t r[FP8 ? FP8_LPW : TILE / NWAVE];  // bf16: this wave's rows (uniform); fp8: per lane
        int32_t rope;                             // bf16: row of this lane's RoPE chunk
    };
    const int my_loads = FP8 ? (wave < L::LOADS - NWAVE * (FP8_LPW - 1) ? FP8_LPW : FP8_LPW - 1) : L::LPW;
    // 656-B rows: lane chunk c16 = 64 k + lane of load k = wave + 4 i lies in
    // row rt = c16 / 41 of the tile, at chunk c = c16 - 41 rt.  Both are fixed
    // per lane and load, so they are computed once and packed in one register:
    // bits 0..15 the byte offset of the row's id in the row list (rt clamped
    // to 31: the last load's spare lanes read chunks c < 32 of row 31 into the
    // slot padding), bits 16..31 the chunk's byte offset in the row.
    uint32_t f_rc[FP8_LPW] = {};
    if constexpr (L::F16) {
#pragma unroll
        for (int i = 0; i < FP8_LPW; ++i) {
            const unsigned c16 = 64 * (wave + NWAVE * i) + lane;
            const unsigned rt = c16 / 41u;
            f_rc[i] = 4u * (rt < TILE - 1 ? rt : TILE - 1) | (16u * (c16 - 41u * rt)) << 16;
        }
    }
    auto load_rows = [&](int ti) -> GatherRows {
        const LDS_AS int32_t* rows = s_rows + ti * TILE;
        const int ln = opaque(lane);
        GatherRows g;
        if constexpr (!FP8) {
            // the wave's 8 row ids: two 16-byte reads (32-byte aligned)
            const u32x4 ra = lds_ld<u32x4>((lds_cptr)(rows + 8 * wave));
            const u32x4 rb = lds_ld<u32x4>((lds_cptr)(rows + 8 * wave + 4));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                g.r[i] = __builtin_amdgcn_readfirstlane((int)ra[i]);
                g.r[4 + i] = __builtin_amdgcn_readfirstlane((int)rb[i]);
            }
            g.rope = rows[8 * wave + (ln >> 3)];
        } else {
#pragma unroll
            for (int i = 0; i < FP8_LPW; ++i) {
                if constexpr (L::MX) {
                    const int k = wave + NWAVE * i;                      // load of the tile (uniform)
                    g.r[i] = rows[k < 16 ? 2 * k + (ln >> 5) : (k < 20 ? 8 * (k - 16) + (ln >> 3) : (ln & 31))];
                } else {
                    // (an opaque copy: the unpacked halves would be hoisted out of the loop)
                    g.r[i] = lds_ld<int32_t>((lds_cptr)rows + ((unsigned)opaque((int)f_rc[i]) & 0xFFFFu));
                }
            }
            g.rope = 0;
        }
        return g;
    };
    // i-th load of this wave for a tile
    auto issue_one = [&](const GatherRows& g, int slot, int i) {
        const int ln = opaque(lane);
        if constexpr (!FP8) {
            const lds_ptr tb = slot_buf(slot);
            if (i < 8) {
                const int r = 8 * wave + i;
                // wave-uniform row: the row address is scalar, the lane part a
                // 32-bit offset.  Row ids are valid (>= 0) and the row stride
                // is below 4 GiB (checked on the host), so the row's byte
                // offset is an unsigned 32 x 32-bit product: four scalar
                // instructions, where a signed 64-bit product takes nine, and
                // with one wave per SIMD they issue one at a time in the
                // gather burst after the tile barrier.
                // (V4 rows: the row stride is 2 x an int32 element count)
                const unsigned char* base;
                if constexpr (L::D512) {
                    const int32_t id = g.r[i];
                    base = (dsa_rows::row_in_pool2(id) ? p.kv2 : p.kv) +
                           (uint64_t)(uint32_t)dsa_rows::row_index(id) * (uint32_t)p.row_bytes;
                } else {
                    base = p.kv + (uint64_t)(uint32_t)g.r[i] * (uint32_t)p.row_bytes;
                }
                lds_dma16_s(base, 16u * (unsigned)(ln ^ nope_sw(r)), tb + r * NOPE_STRIDE);
            } else if constexpr (!L::D512) {
                const int r = 8 * wave + (ln >> 3);
                const unsigned char* src = p.kv + (uint64_t)(uint32_t)g.rope * (uint32_t)p.row_bytes + 2 * D_NOPE +
                                           16 * ((ln & 7) ^ rope_sw(r));
                lds_dma16(src, tb + ROPE_OFF + 8 * wave * 128);
            }
        } else {
            if (i < my_loads) {
                // Lane chunk c16 = 41 * rt + c of the raw tile.  The last load
                // runs past the tile's 1312 chunks: those lanes read chunks of
                // row 31 (rt clamped to 31 when the row id was fetched, c
                // < 32) into the slot's padding, so no lane is masked off.
                const int k = wave + NWAVE * i;
                const uint64_t row = (uint32_t)g.r[i];
                if constexpr (L::V4MX) {
                    // NoPE (with its scales) or RoPE stream of the row's pool;
                    // a row of the second (extend) pool carries the POOL2 tag.
                    // The pool pointers pass through registers the compiler
                    // cannot trace to the argument block: a per-lane choice
                    // between two argument fields otherwise becomes a per-lane
                    // load of the field, whose vmcnt wait drains the gathers.
                    const unsigned char* n0 = p.kv;
                    const unsigned char* n1 = p.kv2;
                    const unsigned char* q0 = p.kv_ro;
                    const unsigned char* q1 = p.kv2_ro;
                    asm("" : "+s"(n0), "+s"(n1), "+s"(q0), "+s"(q1));
                    const bool e2 = dsa_rows::row_in_pool2(g.r[i]);
                    const uint64_t r64 = (uint32_t)dsa_rows::row_index(g.r[i]);
                    const unsigned char* src =
                        k < 16 ? (e2 ? n1 : n0) + r64 * p.kvn_st + 16 * (ln & 31)
                               : (e2 ? q1 : q0) + r64 * p.kvr_st + 16 * (ln & 7);
                    lds_dma16(src, RING + slot * RAW_STRIDE + 1024 * k);
                } else if constexpr (L::MX) {
                    // one stream per load: base and row stride are wave-uniform;
                    // lane ln's piece is the one its slot position holds (the
                    // permutation above)
                    const int rn = 2 * k + (ln >> 5), rr = 8 * (k - 16) + (ln >> 3);
                    const unsigned char* src =
                        k < 16 ? p.kv + row * p.kvn_st + 16 * ((ln & 31) ^ (rn & 15))
                               : (k < 20 ? p.kv_ro + row * p.kvr_st + 16 * ((ln & 7) ^ (rr & 7))
                                         : p.kv_sc + row * p.kvs_st);
                    lds_dma16(src, RING + slot * RAW_STRIDE + 1024 * k);
                } else {
                    lds_dma16(p.kv + (row * (uint32_t)p.row_bytes + ((unsigned)opaque((int)f_rc[i]) >> 16)),
                              RING + slot * RAW_STRIDE + 1024 * k);
                }
            }
        }
    };
    auto issue_rows = [&](const GatherRows& g, int slot) {
#pragma unroll
        for (int i = 0; i < L::LPW; ++i) issue_one(g, slot, i);
    };
    // wait until this wave's loads of all but the newest `keep` tiles landed
    auto wait_tiles = [&](int keep) {
        if (keep <= 0) wait_vm<0>();
        else if constexpr (FP8) {
            if (keep == 1) { if (my_loads == FP8_LPW) wait_vm<FP8_LPW>(); else wait_vm<FP8_LPW - 1>(); }
            else { if (my_loads == FP8_LPW) wait_vm<2 * FP8_LPW>(); else wait_vm<2 * (FP8_LPW - 1)>(); }
        } else {
            if (keep == 1) wait_vm<L::LPW>();
            else wait_vm<2 * L::LPW>();
        }
    };

    // ---- 3. fp8: dequantise a raw slot into a tile buffer (cooperative) ----
    // Nine pieces per tile.  Pieces 0..7: wave w converts row w + 4j; lane l
    // owns NoPE codes 8l..8l+7.  656-B rows (scale group l/16): fp16 =
    // fp16(code * 2^e) * fp16(mantissa) where scale = mantissa * 2^e.  MXFP8
    // rows (E8M0 block l/4): bf16 = code * 2^(e - 127), exact.  Piece 8:
    // RoPE, copied as bf16 (one 16-byte chunk per thread).
    auto deq_load = [&](lds_cptr rb, int j) -> DeqPiece {
        const int ln = opaque(lane);
        DeqPiece d;
        if (j < TILE / NWAVE) {
            const int r = wave + NWAVE * j;
            const lds_cptr rr = rb + r * (L::MX ? D_NOPE : FP8_ROW);
            if constexpr (L::V4MX) {
                // lanes 0..55: codes 8l..8l+7, then the 8 scale bytes holding
                // block l/4; lanes 56..63: RoPE values 8(l-56)..+7 (bf16) in
                // two halves.  Same two loads on every lane: no branch.
                const bool rp = ln >= 56;
                const lds_cptr ra = rb + MX_ROPE_OFF + 128 * r + 16 * (ln & 7);
                const u32x2 lo = lds_ld<u32x2>(rp ? ra : rr + 8 * ln);
                const u32x2 hi8 = lds_ld<u32x2>(rp ? ra + 8 : rr + DSA_MLA_V4_NOPE + 8 * (ln >> 5));
                d.v = u32x4{lo[0], lo[1], hi8[0], hi8[1]};
                return d;
            }
            // (MXFP8: codes 8 ln.. are in piece ln / 2, at its permuted position)
            const u32x2 codes = lds_ld<u32x2>(L::MX ? rr + 16 * ((ln >> 1) ^ (r & 15)) + 8 * (ln & 1) : rr + 8 * ln);
            d.v[0] = codes[0];
            d.v[1] = codes[1];
            if constexpr (L::MX) {
                d.v[2] = lds_ld<unsigned char>(rb + MX_SC_OFF + 16 * r + (ln >> 2));
                d.v[3] = 0;
            } else {
                d.v[2] = __float_as_uint(lds_ld<float>(rr + FP8_SCALE_OFF + 4 * (ln >> 4)));
                d.v[3] = 0;
            }
        } else {
            const int t8 = opaque(tid);
            if constexpr (L::MX)
                d.v = lds_ld<u32x4>(rb + MX_ROPE_OFF + (t8 >> 3) * 128 + 16 * (t8 & 7));
            else
                d.v = lds_ld<u32x4>(rb + (t8 >> 3) * FP8_ROW + FP8_ROPE_OFF + 16 * (t8 & 7));
        }
        return d;
    };
    // 656-B rows: set when a dequantised piece's scale is outside the fp16
    // path's range (FP8_SCALE_LIMIT_BITS); range_bad collects it over the
    // tiles that hold list rows.
    bool deq_bad = false, range_bad = false;
    auto deq_store = [&](lds_ptr tb, int j, const DeqPiece& d) {
        const int ln = opaque(lane);
        if (j < TILE / NWAVE) {
            const int r = wave + NWAVE * j;
            if constexpr (L::V4MX) {
                const uint64_t sc8 = ((uint64_t)d.v[3] << 32) | d.v[2];
                const unsigned e = (unsigned)(sc8 >> (8 * ((ln >> 2) & 7))) & 0xFFu;
                const u32x4 cv = mx_to_bf16(d.v[0], d.v[1], e);
                lds_st<u32x4>(tb + r * NOPE_STRIDE + 16 * (ln ^ nope_sw(r)), ln >= 56 ? d.v : cv);
                return;
            } else if constexpr (L::MX) {
                lds_st<u32x4>(tb + r * NOPE_STRIDE + 16 * (ln ^ nope_sw(r)), mx_to_bf16(d.v[0], d.v[1], d.v[2]));
                return;
            }
            const float sc = __uint_as_float(d.v[2]);
            deq_bad |= d.v[2] >= FP8_SCALE_LIMIT_BITS;
            const _Float16 m16 = (_Float16)__uint_as_float((d.v[2] & 0x007FFFFFu) | 0x3F800000u);
            const f16x2 mm = {m16, m16};
            const f16x2 h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)d.v[0], sc, false) * mm;
            const f16x2 h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)d.v[0], sc, true) * mm;
            const f16x2 h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)d.v[1], sc, false) * mm;
            const f16x2 h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)d.v[1], sc, true) * mm;
            const u32x4 out = {__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1),
                               __builtin_bit_cast(unsigned, h2), __builtin_bit_cast(unsigned, h3)};
            lds_st<u32x4>(tb + r * NOPE_STRIDE + 16 * (ln ^ nope_sw(r)), out);
        } else {
            const int t8 = opaque(tid);
            const int r = t8 >> 3, c = t8 & 7;
            lds_st<u32x4>(tb + ROPE_OFF + 128 * r + 16 * (c ^ rope_sw(r)), d.v);
        }
    };
    auto dequant = [&](lds_cptr rb, lds_ptr tb) {
#pragma unroll
        for (int j = 0; j < (L::D512 || L::SQK ? DEQ_PIECES - 1 : DEQ_PIECES); ++j) deq_store(tb, j, deq_load(rb, j));
    };
    // The same NoPE dequant split by output dims (656-B rows, MXFP8 V3.2):
    // piece g = 4u + m of wave w is rows 16u .. 16u + 15, dims
    // 128w + 32m .. +31 - exactly the V block that PV group (u, m) of wave w
    // reads; lane l converts row 16u + l/4, dims d0 = 128w + 32m + 8(l % 4)
    // .. +7.  A wave writes only dims it reads itself in PV, so a tile buffer
    // is refilled by its own PV readers, each piece once that wave has read it.
    auto deqd_load = [&](lds_cptr rb, int g) -> DeqPiece {
        const int ln = opaque(lane);
        const int r = 16 * (g >> 2) + (ln >> 2);
        const int d0 = 128 * wave + 32 * (g & 3) + 8 * (ln & 3);
        DeqPiece d;
        u32x2 codes;
        if constexpr (L::MX) {
            // piece d0 / 16 of the row, at its permuted position
            codes = lds_ld<u32x2>(rb + D_NOPE * r + 16 * ((d0 >> 4) ^ (r & 15)) + 8 * ((d0 >> 3) & 1));
            d.v[2] = lds_ld<unsigned char>(rb + MX_SC_OFF + 16 * r + (d0 >> 5));
        } else {
            const lds_cptr rr = rb + r * FP8_ROW;
            codes = lds_ld<u32x2>(rr + d0);
            d.v[2] = __float_as_uint(lds_ld<float>(rr + FP8_SCALE_OFF + 4 * wave));
        }
        d.v[0] = codes[0];
        d.v[1] = codes[1];
        d.v[3] = 0;
        return d;
    };
    auto deqd_store = [&](lds_ptr tb, int g, const DeqPiece& d) {
        const int ln = opaque(lane);
        const int r = 16 * (g >> 2) + (ln >> 2);
        const int ch = 16 * wave + 4 * (g & 3) + (ln & 3);    // 16-byte chunk: dims 8 ch .. 8 ch + 7
        u32x4 out;
        if constexpr (L::MX) {
            out = mx_to_bf16(d.v[0], d.v[1], d.v[2]);
        } else {
            const float sc = __uint_as_float(d.v[2]);
            const _Float16 m16 = (_Float16)__uint_as_float((d.v[2] & 0x007FFFFFu) | 0x3F800000u);
            const f16x2 mm = {m16, m16};
            const f16x2 h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)d.v[0], sc, false) * mm;
            const f16x2 h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)d.v[0], sc, true) * mm;
            const f16x2 h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)d.v[1], sc, false) * mm;
            const f16x2 h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)d.v[1], sc, true) * mm;
            out = u32x4{__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1),
                        __builtin_bit_cast(unsigned, h2), __builtin_bit_cast(unsigned, h3)};
        }
        lds_st<u32x4>(tb + r * NOPE_STRIDE + 16 * (ch ^ nope_sw(r)), out);
    };

    // ---- online softmax state (fixed reference max) ----
    // p = exp2(s*c - m_ref) with m_ref fixed for the whole pass (the first
    // tile's maximum per head), so the O accumulators are never rescaled in
    // the loop.  The pass also tracks the largest raw score per head; if it
    // exceeds the reference by more than TAU (log2 units: some p left the
    // range of the P format) the workgroup reruns its tiles once with m_ref
    // set to that exact maximum, where every p <= 1.  A second rerun never
    // happens (the maximum is exact), and none is allowed, so no input -
    // NaN, infinities or scores far beyond fp32's integer range included -
    // can keep the loop going.
    // (656-B rows: per head, times the power of two that brought its Q into
    // fp16's range, see convert_q)
    float c_s = p.scale_log2;
    // O^T accumulators of this wave: dims 128*wave + 32*m + (0..31) for the
    // 32 heads 32*h + (0..31): o[4*m + h] (the PV step is split by output
    // dims across the waves, so each gathered V value is read by one wave).
    f32x16 o[D_VO / 32];
    float m_ref = 0.0f, l_lane = 0.0f, s_max = -INFINITY;
    // Q conversion, once its loads have landed
    auto convert_q = [&]() {
        if constexpr (L::F16) {
            // The NoPE part of Q is converted to fp16 for the fp16 MFMAs.  A
            // head with |q| >= 2^15 would leave fp16's range: the whole head
            // (NoPE and RoPE) is scaled by 2^-k, bringing its largest NoPE
            // value below 2^15, and c_s by 2^k, so the scaled scores are the
            // same.  Both are exact; k = 0 for every |q| < 2^15.
            typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
            u16x2 amax = {0, 0};
#pragma unroll
            for (int ks = 0; ks < KS_NOPE; ++ks)
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    amax = __builtin_elementwise_max(amax, __builtin_bit_cast(u16x2, qf[ks][w] & 0x7FFF7FFFu));
            // biased exponent of the head's largest |q| (bf16 bits >> 7)
            int eb = max((int)amax[0], (int)amax[1]) >> 7;
            eb = max(eb, __shfl_xor(eb, 32, 64));
            const int k = max(eb - 141, 0);                   // 141 = 127 + 14
            const float s = __uint_as_float((unsigned)(127 - k) << 23);
            c_s = p.scale_log2 * __uint_as_float((unsigned)(127 + k) << 23);
#pragma unroll
            for (int ks = 0; ks < KS_NOPE; ++ks)
#pragma unroll
                for (int w = 0; w < 4; ++w) qf[ks][w] = bf16x2_to_f16x2(qf[ks][w], s);
#pragma unroll
            for (int ks = KS_NOPE; ks < KS_ALL; ++ks)
#pragma unroll
                for (int w = 0; w < 4; ++w) qf[ks][w] = bf16x2_scale(qf[ks][w], s);
        } else if constexpr (L::SQK) {
            // the codes stay fp8; the scale operands take, per lane, the bytes
            // of blocks 2 k8 + hi: the even (hi = 0) or odd bytes of the 16
            q_sc8[0] = __builtin_amdgcn_perm(q_scales[1], q_scales[0], hi ? 0x07050301u : 0x06040200u);
            q_sc8[1] = __builtin_amdgcn_perm(q_scales[3], q_scales[2], hi ? 0x07050301u : 0x06040200u);
        } else if constexpr (L::MX) {
            // fp8 NoPE of Q -> bf16: dims 16ks + 8hi .. +7 lie in scale block ks / 2
#pragma unroll
            for (int ks = 0; ks < L::Q8_KS; ++ks) {
                const unsigned e = (q_scales[ks >> 3] >> (8 * ((ks >> 1) & 3))) & 0xFFu;
                qf[ks] = mx_to_bf16(qf[ks][0], qf[ks][1], e);
            }
        }
    };
    constexpr int NPRE = FP8 ? 3 : 2;       // tiles in flight before a chunk's loop
    GatherRows gnext;

    // P values -> MFMA operand (fp16 for the 656-B cache, else bf16)
    auto to_p = [&](const float* e) -> u32x4 {
        u32x4 pb;
        if constexpr (L::F16) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const f16x2 h = {(_Float16)e[2 * w], (_Float16)e[2 * w + 1]};
                pb[w] = __builtin_bit_cast(unsigned, h);
            }
        } else {
            const f32x8 a = {e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]};
            pb = __builtin_bit_cast(u32x4, __builtin_convertvector(a, bf16x8));
        }
        return pb;
    };

    // Padding rows of a list's last tile get no weight.  Lane (hi, r32), reg r
    // holds row 8*(r/4) + 4*hi + r%4.  Only the last tile takes the branch; the
    // empty asm keeps the compiler from turning it into selects (and hoisted
    // row numbers) that every tile would pay for.
    auto mask_rows = [&](f32x16& s, int rows_left) {
        if (rows_left < TILE) {
            asm volatile("");
            const int h4 = 4 * opaque(hi);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 8 * (r >> 2) + h4 + (r & 3);
                s[r] = row < rows_left ? s[r] : -INFINITY;
            }
        }
    };
    // the largest score of a list's first tile (rows below rows_left)
    auto first_max = [&](const f32x16& s, int rows_left) -> float {
        asm volatile("");
        const int h4 = 4 * opaque(hi);
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r >> 2) + h4 + (r & 3);
            mx = fmaxf(mx, row < rows_left ? s[r] : -INFINITY);
        }
        return fmaxf(mx, __shfl_xor(mx, 32, 64));
    };

    // ---- S^T = K Q^T of the tile in buffer kt (32 rows x this wave's 32 heads) ----
    // Software pipeline pinned with scheduling barriers: the K fragment of
    // k-step ks+KPF is read while MFMA ks runs.
    auto qk = [&](lds_cptr kt, auto&& per_step) -> f32x16 {
        const int ln = lane;
        const int lhi = ln >> 5, lr = ln & 31;
        // K fragment of k-step ks (A operand of S^T = K Q^T): row lr, chunk 2ks+hi
        const lds_cptr k_even = kt + lr * NOPE_STRIDE + 16 * (lhi ^ nope_sw(lr));
        const lds_cptr k_odd = kt + lr * NOPE_STRIDE + 16 * ((2 + lhi) ^ nope_sw(lr));
        const lds_cptr k_rope = kt + ROPE_OFF + 128 * lr;
        const int rsw = rope_sw(lr);
        // K prefetch depth, per format by measurement (deeper spilled or ran slower)
        constexpr int KPF = L::V4MX ? 4 : (L::MX ? 3 : (FP8 ? 4 : 6));
        auto k_addr = [&](int ks) -> lds_cptr {
            return ks < KS_NOPE ? ((ks & 1) ? k_odd : k_even) + 64 * (ks >> 1)
                                : k_rope + 16 * ((2 * (ks - KS_NOPE) + lhi) ^ rsw);
        };
        u32x4 kb[KPF];
#pragma unroll
        for (int i = 0; i < KPF; ++i) kb[i] = lds_ld<u32x4>(k_addr(i));
        // one accumulator chain: back-to-back dependent MFMAs issue at the full
        // rate, and two chains would cost 16 adds per tile to combine
        f32x16 acc = {};
#pragma unroll
        for (int ks = 0; ks < L::KS; ++ks) {
            __builtin_amdgcn_sched_barrier(0);
            if (L::F16 && ks < KS_NOPE) acc = mfma_f16(kb[ks % KPF], qf[ks], acc);
            else acc = mfma_bf16(kb[ks % KPF], qf[ks], acc);
            if (ks + KPF < L::KS) kb[ks % KPF] = lds_ld<u32x4>(k_addr(ks + KPF));
            per_step(ks);
        }
        __builtin_amdgcn_sched_barrier(0);
        return acc;
    };

    // ---- MXFP8 (V3.2) S^T = K Q^T straight from the raw slot of the tile ----
    // NoPE: 8 scaled fp8 MFMAs (v_mfma_scale_f32_32x32x64_f8f6f4, 64-deep):
    // lane (hi, lr) holds row lr's codes 64 k8 + 16 hi .. +15 and
    // 64 k8 + 32 + 16 hi .. +15, and its scale byte k8 % 4 of k_sc8[k8 / 4] is
    // row lr's E8M0 of block 2 k8 + hi (Q the same way); the MFMA applies
    // both scales per 32-block.  RoPE: 4 bf16 MFMAs from the raw RoPE stream.
    auto qk8 = [&](lds_cptr raw, auto&& per_step) -> f32x16 {
        const int ln = lane;
        const int lhi = ln >> 5, lr = ln & 31;
        const lds_cptr kn = raw + lr * D_NOPE;
        const int sw = lr & 15;
        const u32x4 ksc = lds_ld<u32x4>(raw + MX_SC_OFF + 16 * lr);
        auto k_frag = [&](int k8) -> i32x8 {
            const u32x4 a0 = lds_ld<u32x4>(kn + 16 * ((4 * k8 + lhi) ^ sw));
            const u32x4 a1 = lds_ld<u32x4>(kn + 16 * ((4 * k8 + 2 + lhi) ^ sw));
            return __builtin_bit_cast(i32x8, __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7));
        };
        auto q_frag = [&](int k8) -> i32x8 {
            return __builtin_bit_cast(i32x8, __builtin_shufflevector(qf[2 * k8], qf[2 * k8 + 1], 0, 1, 2, 3, 4, 5, 6, 7));
        };
        i32x8 kb[2] = {k_frag(0), k_frag(1)};
        const unsigned sel = lhi ? 0x07050301u : 0x06040200u;
        const int k_sc8[2] = {(int)__builtin_amdgcn_perm(ksc[1], ksc[0], sel), (int)__builtin_amdgcn_perm(ksc[3], ksc[2], sel)};
        f32x16 acc = {};
#pragma unroll
        for (int k8 = 0; k8 < KS_NOPE / 4; ++k8) {
            __builtin_amdgcn_sched_barrier(0);
            acc = mfma_scale8(k8 & 3, kb[k8 & 1], q_frag(k8), acc, k_sc8[k8 >> 2], (int)q_sc8[k8 >> 2]);
            if (k8 + 2 < KS_NOPE / 4) kb[k8 & 1] = k_frag(k8 + 2);
            per_step(k8);
        }
        const lds_cptr kr = raw + MX_ROPE_OFF + 128 * lr;
        const int rsw = lr & 7;
        u32x4 rb[2] = {lds_ld<u32x4>(kr + 16 * (lhi ^ rsw)), lds_ld<u32x4>(kr + 16 * ((2 + lhi) ^ rsw))};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            acc = mfma_bf16(rb[j & 1], qf[KS_NOPE + j], acc);
            if (j + 2 < 4) rb[j & 1] = lds_ld<u32x4>(kr + 16 * ((2 * (j + 2) + lhi) ^ rsw));
        }
        __builtin_amdgcn_sched_barrier(0);
        return acc;
    };

    // ---- fp8 caches, one tile: QK^T (after the gathers of a later tile), softmax, PV (+ dequant of the next tile) ----
    // kt: buffer holding tile `it`; nxt: buffer receiving tile it+1.
    bool first_tile = true;
    auto step = [&](int it, lds_cptr kt, lds_ptr nxt) {
        const int ln = opaque(lane);
        const int lhi = ln >> 5;
        const bool do_issue = it + NPRE < ntiles;
        const int issue_slot = FP8 ? it % 3 : (it + 2) % 3;
        const GatherRows gcur = gnext;
        deq_bad = false;
        __builtin_amdgcn_sched_barrier(0);
        // Gathers of tile it+NPRE, all at once: the tile barrier just before
        // has drained this wave's LDS accesses, and an LDS-DMA load issued
        // while LDS reads are in flight holds the wave far longer.
        // (MXFP8 V3.2: after the P barrier, into this tile's own raw slot)
        if constexpr (!L::SQK)
            if (do_issue) issue_rows(gcur, issue_slot);
        __builtin_amdgcn_sched_barrier(0);
        // V4 fp8 rows: the next tile's dequant runs between the QK^T MFMAs
        // (piece j loads at k-step 4j, is converted and stored at 4j + 2):
        // measured 2 % faster there, neutral for the other fp8 formats, which
        // keep it between the PV MFMAs
        constexpr bool DEQ_QK = L::V4MX;
        DeqPiece dq[2];
        const lds_cptr draw = FP8 ? RING + ((it + 1) % 3) * RAW_STRIDE : kt;
        constexpr int NPIECE = L::D512 ? DEQ_PIECES - 1 : DEQ_PIECES;
        // MXFP8 V3.2: K straight from this tile's raw slot (scaled fp8 MFMAs)
        f32x16 sacc = [&]() -> f32x16 {
            if constexpr (L::SQK) {
                return qk8(RING + (it % 3) * RAW_STRIDE, [](int) {});
            } else {
                return qk(kt, [&](int ks) {
                    if constexpr (DEQ_QK) {
                        if ((ks & 3) == 0 && ks / 4 < NPIECE) dq[(ks / 4) & 1] = deq_load(draw, ks / 4);
                        if ((ks & 3) == 2 && ks / 4 < NPIECE) deq_store(nxt, ks / 4, dq[(ks / 4) & 1]);
                    }
                });
            }
        }();
        // row ids of the tile issued in the next step
        if (it + NPRE + 1 < ntiles) gnext = load_rows(it + NPRE + 1);

        // ---- softmax numerators -> P (this wave's 32 heads) ----
        // lane (hi, r32), reg r holds row 8*(r/4) + 4*hi + r%4 of head r32:
        // regs 0..7 are rows 0..15 (PV k-step u = 0), regs 8..15 rows 16..31.
        const int rows_left = n_valid - it * TILE;
        if (first_tile) {
            m_ref = first_max(sacc, rows_left) * c_s;
            first_tile = false;
        }
        mask_rows(sacc, rows_left);
        if (nchunks == 1 && ntiles == 1 && it == 0) {
            // Single-tile list: fold the exact sum into the reference, so
            // that p = exp2(s - m_ref) is already normalised when it is
            // rounded - the order the reference uses
            // (opus_attn/dsa_v32/common/host.cc:448-451); with few rows the
            // outputs are large and a different rounding order would show.
            // (an attention sink joins the sum: mla_v4_host.cc:469-472)
            float lt = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) lt += __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], c_s, -m_ref));
            lt += __shfl_xor(lt, 32, 64);
            float m_fold = m_ref;
            if constexpr (L::D512)
                if (p.attn_sink) add_sink(lt, m_ref, p.attn_sink[head_q] * LOG2E, lt, m_fold);
            m_ref = m_fold + __builtin_amdgcn_logf(lt);
        }
        // P of both halves, then one barrier: the wave's VALU work does not
        // overlap its own MFMAs, so exponentials placed between the PV MFMAs
        // would save nothing and a second barrier would cost one.
        float e[16];
        auto p_exp = [&](int r) { e[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], c_s, -m_ref)); };
        auto p_store = [&](int u) {
            float lt = 0.0f, sm = -INFINITY;
#pragma unroll
            for (int r = 8 * u; r < 8 * u + 8; ++r) {
                lt += e[r];
                sm = fmaxf(sm, sacc[r]);
            }
            l_lane += lt;
            s_max = fmaxf(s_max, sm);
            lds_st<u32x4>(PX + ((u * NWAVE + wave) * 64 + ln) * 16, to_p(e + 8 * u));
        };
#pragma unroll
        for (int r = 0; r < 16; ++r) p_exp(r);
        p_store(0);
        p_store(1);
        tile_barrier();     // every wave's P is visible
        if constexpr (L::SQK) {
            // every wave is done with this tile's raw slot: refill it
            __builtin_amdgcn_sched_barrier(0);
            if (do_issue) issue_rows(gcur, issue_slot);
            __builtin_amdgcn_sched_barrier(0);
        }

        // ---- O^T[128 dims of this wave x 128 heads] += V^T P^T ----
        // Transposed V reads: 16-lane group g16 reads rows R..R+3 (lane
        // 4rr+pp: row R+rr, dims d0+4pp..+3) with R = 16u + 4hi and R + 8.
        // 656-B and MXFP8 rows: the dequant of the next tile runs between
        // these MFMAs (V4 fp8 rows: between the QK^T MFMAs above).
        {
            const int g16 = ln >> 4, i16 = ln & 15, rr = i16 >> 2, pp = i16 & 3;
            const int vx = 2 * (g16 & 1) + (pp >> 1);
            const lds_cptr v_a = kt + (4 * lhi + rr) * NOPE_STRIDE + 16 * (vx ^ lhi) + 8 * (pp & 1) + 256 * wave;
            const lds_cptr v_b = kt + (4 * lhi + rr + 8) * NOPE_STRIDE + 16 * (vx ^ (lhi + 2)) + 8 * (pp & 1) + 256 * wave;
            auto v_frag = [&](int u, int m) -> u32x4 {
                const s16x4 va = lds_read_tr16(v_a + 16 * u * NOPE_STRIDE + 64 * m);
                const s16x4 vb = lds_read_tr16(v_b + 16 * u * NOPE_STRIDE + 64 * m);
                return __builtin_bit_cast(u32x4, __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7));
            };
            int step_i = 0;   // MFMA-group counter (8 groups of 4 MFMAs)
            // P fragments of half u; those of half 1 and its first V fragment
            // are read in the last MFMA group of half 0
            u32x4 pbf[NWAVE], pnx[NWAVE];
#pragma unroll
            for (int h = 0; h < NWAVE; ++h) pbf[h] = lds_ld<u32x4>(PX + (h * 64 + ln) * 16);
            u32x4 va_cur = v_frag(0, 0);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    __builtin_amdgcn_sched_barrier(0);
                    u32x4 va_nxt = va_cur;
                    if (m + 1 < 4) {
                        va_nxt = v_frag(u, m + 1);
                    } else if (u == 0) {
#pragma unroll
                        for (int h = 0; h < NWAVE; ++h) pnx[h] = lds_ld<u32x4>(PX + ((NWAVE + h) * 64 + ln) * 16);
                        va_nxt = v_frag(1, 0);
                    }
#pragma unroll
                    for (int h = 0; h < NWAVE; ++h) mfma_o<L::F16>(o[4 * m + h], va_cur, pbf[h]);
                    if constexpr (FP8 && !DEQ_QK) {
                        // piece j: loads in MFMA group j, conversion + store in group j+1
                        const int j = step_i;
                        dq[j & 1] = deq_load(draw, j);
                        if (j >= 1) deq_store(nxt, j - 1, dq[(j - 1) & 1]);
                    }
                    va_cur = va_nxt;
                    ++step_i;
                }
                if (u == 0) {
#pragma unroll
                    for (int h = 0; h < NWAVE; ++h) pbf[h] = pnx[h];
                }
            }
            if constexpr (FP8 && !DEQ_QK) {
                // pieces 0..7 were loaded in the 8 MFMA groups, 0..6 stored
                static_assert(DEQ_PIECES == 9, "dequant pieces vs MFMA groups");
                __builtin_amdgcn_sched_barrier(0);
                deq_store(nxt, 7, dq[1]);
                // RoPE block (MXFP8 V3.2: QK^T reads it from the raw slot)
                if constexpr (!L::D512 && !L::SQK) deq_store(nxt, 8, deq_load(draw, 8));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // (past the last tile the dequant converted a stale slot: not counted)
        if constexpr (L::F16)
            if (it + 1 < ntiles) range_bad |= deq_bad;
    };

    // ---- bf16 caches: a software-pipelined tile loop ----
    // Iteration it computes QK^T of tile it+1, then PV of tile it with the
    // softmax numerators of tile it+1 worked out between its MFMAs, and stores
    // tile it+1's P into the other P buffer; the next iteration's barrier
    // publishes it, so a tile costs one workgroup barrier.  The arithmetic and
    // its order per tile are those of `step` (QK^T, p = exp2(s c - m_ref), the
    // sums per half, the O accumulation order): both loops give the same bits.
    // Padding rows of the last tile, and the raw maximum of the pass.
    auto mask_track = [&](f32x16& s, int j) {
        mask_rows(s, n_valid - j * TILE);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float sm = -INFINITY;
#pragma unroll
            for (int r = 8 * u; r < 8 * u + 8; ++r) sm = fmaxf(sm, s[r]);
            s_max = fmaxf(s_max, sm);
        }
    };
    // P of a tile from its numerators, half u (rows 16u..16u+15) into P buffer px;
    // half 0 before half 1, so the sums accumulate in the same order as in `step`
    auto p_half = [&](const float* e, int u, lds_ptr px) {
        const int ln = opaque(lane);
        float lt = 0.0f;
#pragma unroll
        for (int r = 8 * u; r < 8 * u + 8; ++r) lt += e[r];
        l_lane += lt;
        lds_st<u32x4>(px + ((u * NWAVE + wave) * 64 + ln) * 16, to_p(e + 8 * u));
    };
    // tile 0 of a pass: the reference (first pass), padding, the one-tile fold, P
    auto soft_first = [&](f32x16& s, lds_ptr px) {
        if (first_tile) {
            m_ref = first_max(s, n_valid) * c_s;
            first_tile = false;
        }
        mask_track(s, 0);
        if (nchunks == 1 && ntiles == 1) {
            float lt = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) lt += __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c_s, -m_ref));
            lt += __shfl_xor(lt, 32, 64);
            float m_fold = m_ref;
            if constexpr (L::D512)
                if (p.attn_sink) add_sink(lt, m_ref, p.attn_sink[head_q] * LOG2E, lt, m_fold);
            m_ref = m_fold + __builtin_amdgcn_logf(lt);
        }
        float e[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c_s, -m_ref));
        p_half(e, 0, px);
        p_half(e, 1, px);
    };
    // O^T += V^T P^T for the tile in kv_t with P from px_cur; with_exp
    // (std::true_type): the numerators of the next tile's scores sn go to en,
    // two per MFMA group (group (u, m) gives en[8u + 2m], en[8u + 2m + 1])
    // with_deq (std::true_type): piece g = 4u + m of the tile in raw slot draw
    // is dequantised into tbd (kv_t itself) in group (u, m), stored after the
    // group's MFMAs have consumed this wave's V block (u, m)
    auto pv_pipe = [&](lds_cptr kv_t, lds_cptr px_cur, const f32x16& sn, float* en, auto with_exp,
                       lds_cptr draw, lds_ptr tbd, auto with_deq) {
        const int ln = lane;
        const int lhi = ln >> 5;
        const int g16 = ln >> 4, i16 = ln & 15, rr = i16 >> 2, pp = i16 & 3;
        const int vx = 2 * (g16 & 1) + (pp >> 1);
        const lds_cptr v_a = kv_t + (4 * lhi + rr) * NOPE_STRIDE + 16 * (vx ^ lhi) + 8 * (pp & 1) + 256 * wave;
        const lds_cptr v_b = kv_t + (4 * lhi + rr + 8) * NOPE_STRIDE + 16 * (vx ^ (lhi + 2)) + 8 * (pp & 1) + 256 * wave;
        auto v_frag = [&](int u, int m) -> u32x4 {
            const s16x4 va = lds_read_tr16(v_a + 16 * u * NOPE_STRIDE + 64 * m);
            const s16x4 vb = lds_read_tr16(v_b + 16 * u * NOPE_STRIDE + 64 * m);
            return __builtin_bit_cast(u32x4, __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7));
        };
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            u32x4 pbf[NWAVE];
#pragma unroll
            for (int h = 0; h < NWAVE; ++h) pbf[h] = lds_ld<u32x4>(px_cur + ((u * NWAVE + h) * 64 + ln) * 16);
            u32x4 va_cur = v_frag(u, 0);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                const u32x4 va_nxt = m + 1 < 4 ? v_frag(u, m + 1) : va_cur;
                DeqPiece dq;
                if constexpr (decltype(with_deq)::value) dq = deqd_load(draw, 4 * u + m);
#pragma unroll
                for (int h = 0; h < NWAVE; ++h) mfma_o<L::F16>(o[4 * m + h], va_cur, pbf[h]);
                if constexpr (decltype(with_exp)::value) {
                    const int r0 = 8 * u + 2 * m;
                    en[r0] = __builtin_amdgcn_exp2f(__builtin_fmaf(sn[r0], c_s, -m_ref));
                    en[r0 + 1] = __builtin_amdgcn_exp2f(__builtin_fmaf(sn[r0 + 1], c_s, -m_ref));
                }
                if constexpr (decltype(with_deq)::value) deqd_store(tbd, 4 * u + m, dq);
                va_cur = va_nxt;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    resolve_chunk(0, true);
    for (int pass = 0;; ++pass) {
#pragma unroll
        for (int mb = 0; mb < D_VO / 32; ++mb) o[mb] = f32x16{};
        o_fence(o);
        l_lane = 0.0f;
        s_max = -INFINITY;
        first_tile = pass == 0;
        for (int c = 0; c < nchunks; ++c) {
            // a one-chunk list keeps its row list for the second pass; chunk 0
            // of pass 0 was resolved before the loop (from jv0 / ent0, which
            // are then dead in the tile loop)
            if ((pass == 0 && c > 0) || (pass > 0 && nchunks > 1)) resolve_chunk(c, false);
            // The first tiles' gathers go out with Q possibly still in flight
            // (pass 0, chunk 0).  Loads return in order, so the tile loop's
            // explicit vmcnt waits, which count only gathers, also cover the
            // older Q loads; the compiler's own waits before Q is used count
            // only its loads and so wait for these gathers as well.  In the
            // tile loop the only vector-memory loads are the gathers.
#pragma unroll
            for (int s = 0; s < NPRE; ++s)
                if (s < ntiles) issue_rows(load_rows(s), s);
            if (NPRE < ntiles) gnext = load_rows(NPRE);
            if (pass == 0 && c == 0) convert_q();
            if constexpr (L::SQK) {
                // Pipelined (MXFP8 V3.2).  Iteration j: QK^T of
                // tile j; PV of tile j-1 with tile j's softmax numerators and
                // tile j+1's dequant between its MFMAs (by output dims, into the
                // buffer PV reads: buffer j % 2 holds tile j); a barrier; the
                // gathers of tile j+3 into tile j's raw slot; tile j's P.  K of
                // tile j: buffer j % 2, or (MXFP8) raw slot j % 3.
                auto deq_tile = [&](lds_cptr rb, lds_ptr tb) {
#pragma unroll
                    for (int g = 0; g < 8; ++g) deqd_store(tb, g, deqd_load(rb, g));
                    if constexpr (!L::SQK) deq_store(tb, 8, deq_load(rb, 8));   // RoPE block
                };
                if (ntiles > 0) {
                    wait_tiles(min(ntiles, NPRE) - 1);    // tile 0 landed (1, 2 may be in flight)
                    tile_barrier();
                    deq_tile(RING, T0);
                    // iteration 0: no PV yet; tile 1 is dequantised on its own
                    wait_tiles(2 < ntiles ? 1 : 0);       // tile 1 landed
                    tile_barrier();
                    f32x16 s0 = [&]() -> f32x16 {
                        if constexpr (L::SQK) return qk8(RING, [](int) {});
                        else return qk(T0, [](int) {});
                    }();
                    if (first_tile) {
                        m_ref = first_max(s0, n_valid) * c_s;
                        first_tile = false;
                    }
                    mask_track(s0, 0);
                    if (nchunks == 1 && ntiles == 1) {
                        // one-tile list: the exact sum folded into the reference
                        float lt = 0.0f;
#pragma unroll
                        for (int r = 0; r < 16; ++r) lt += __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], c_s, -m_ref));
                        lt += __shfl_xor(lt, 32, 64);
                        m_ref = m_ref + __builtin_amdgcn_logf(lt);
                    }
                    float e0[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r) e0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], c_s, -m_ref));
                    if (ntiles > 1) deq_tile(RING + RAW_STRIDE, T1);
                    tile_barrier();    // every wave is done with tile 0's raw slot
                    if (NPRE < ntiles) {
                        issue_rows(gnext, 0);
                        if (NPRE + 1 < ntiles) gnext = load_rows(NPRE + 1);
                    }
                    p_half(e0, 0, PX);
                    p_half(e0, 1, PX);
                }
                for (int j = 1; j < ntiles; ++j) {
                    // tile j+1 landed (dequantised below); tile j+2 may be in flight.
                    // The barrier publishes tile j's dequant and tile j-1's P.
                    wait_tiles(j + 2 < ntiles ? 1 : 0);
                    tile_barrier();
                    const lds_ptr tq = (j & 1) ? T1 : T0;     // tile j
                    const lds_ptr tv = (j & 1) ? T0 : T1;     // tile j-1, refilled with tile j+1
                    f32x16 sn = [&]() -> f32x16 {
                        if constexpr (L::SQK) return qk8(RING + (j % 3) * RAW_STRIDE, [](int) {});
                        else return qk(tq, [](int) {});
                    }();
                    mask_track(sn, j);
                    float en[16];
                    // (after the last tile the dequant converts whatever the slot
                    // holds into a buffer that is not read again: no branch
                    // splits the MFMA groups)
                    const lds_cptr dr = RING + ((j + 1) % 3) * RAW_STRIDE;
                    pv_pipe(tv, PX, sn, en, std::true_type{}, dr, tv, std::true_type{});
                    if constexpr (!L::SQK) deq_store(tv, 8, deq_load(dr, 8));   // RoPE block of tile j+1
                    // every wave is done with tile j-1's P and V and tile j's raw slot
                    tile_barrier();
                    if (j + NPRE < ntiles) {
                        __builtin_amdgcn_sched_barrier(0);
                        issue_rows(gnext, (j + NPRE) % 3);
                        __builtin_amdgcn_sched_barrier(0);
                        if (j + NPRE + 1 < ntiles) gnext = load_rows(j + NPRE + 1);
                    }
                    p_half(en, 0, PX);
                    p_half(en, 1, PX);
                }
                if (ntiles > 0) {
                    // the last tile: PV only (its P is published by this barrier)
                    tile_barrier();
                    float en[16];
                    pv_pipe(((ntiles - 1) & 1) ? T1 : T0, PX, f32x16{}, en, std::false_type{}, RING, T0,
                            std::false_type{});
                }
            } else if constexpr (FP8) {
                if (ntiles > 0) {
                    // tile 0 landed (tiles 1, 2 may still be in flight)
                    wait_tiles(min(ntiles, NPRE) - 1);
                    tile_barrier();
                    deq_bad = false;
                    dequant(RING, T0);
                    range_bad |= deq_bad;
                }
                // Two tiles per trip, so that the buffer being read and the one
                // being filled are distinct LDS objects in each step.
                for (int it = 0; it < ntiles; it += 2) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int ii = it + h;
                        if (ii < ntiles) {
                            // tile ii+1 (dequantised in this step) must have landed
                            wait_tiles(ii + 2 < ntiles ? 1 : 0);
                            tile_barrier();
                            step(ii, h == 0 ? T0 : T1, h == 0 ? T1 : T0);
                        }
                    }
                }
            } else {
                // ring slot of tile j: j % 3.  Tiles 0 and 1 were issued above.
                if (ntiles > 0) {
                    wait_tiles(ntiles > 1 ? 1 : 0);    // tile 0 landed
                    tile_barrier();
                    f32x16 s0 = qk(slot_buf(0), [](int) {});
                    soft_first(s0, PX);
                }
                int slot_cur = 0;        // ring slot of tile `it`
                // every tile but the last: QK^T of the next tile, PV of this one
                for (int it = 0; it + 1 < ntiles; ++it) {
                    const int slot_nxt = slot_cur == 2 ? 0 : slot_cur + 1;
                    // tile it+1 landed (the only tile in flight); after the barrier
                    // every wave's P of tile it is visible and every wave is done
                    // with iteration it-1, whose ring slot receives tile it+2
                    wait_vm<0>();
                    tile_barrier();
                    __builtin_amdgcn_sched_barrier(0);
                    if (it + NPRE < ntiles) issue_rows(gnext, slot_nxt == 2 ? 0 : slot_nxt + 1);
                    __builtin_amdgcn_sched_barrier(0);
                    f32x16 sn = qk(slot_buf(slot_nxt), [](int) {});
                    if (it + NPRE + 1 < ntiles) gnext = load_rows(it + NPRE + 1);
                    mask_track(sn, it + 1);
                    float en[16];
                    pv_pipe(slot_buf(slot_cur), PX + (it & 1) * PXB, sn, en, std::true_type{}, RING, T0,
                            std::false_type{});
                    const lds_ptr px_nxt = PX + ((it + 1) & 1) * PXB;
                    p_half(en, 0, px_nxt);
                    p_half(en, 1, px_nxt);
                    slot_cur = slot_nxt;
                }
                if (ntiles > 0) {
                    // the last tile: PV only (its P is published by this barrier)
                    tile_barrier();
                    float en[16];
                    pv_pipe(slot_buf(slot_cur), PX + ((ntiles - 1) & 1) * PXB, f32x16{}, en, std::false_type{}, RING,
                            T0, std::false_type{});
                }
            }
            // drain in-flight gathers before the ring can be reused or left
            wait_vm<0>();
        }
        o_fence(o);
        // per head: the largest score of the pass (log2 units); NaN compares false
        const float top = fmaxf(s_max, __shfl_xor(s_max, 32, 64)) * c_s;
        if (pass == 0 && __builtin_amdgcn_ballot_w64(top - m_ref > L::TAU) != 0 && lane == 0) s_misc[4] = 1;
        if (L::F16 && range_bad) s_misc[5] = 1;
        tile_barrier();
        if (!s_misc[4]) break;
        // new reference: the exact maximum of every score of the head
        m_ref = fmaxf(m_ref, top);
        tile_barrier();              // every wave has read the flag
        if (tid == 0) s_misc[4] = 0;  // visible after the next tile barrier
    }

    // ---- epilogue ----
    // Wave w holds O for dims 128w..128w+127 of all heads; the softmax sums
    // and references are per head, owned by the head's QK wave: exchange them.
    const float l_rows = l_lane + __shfl_xor(l_lane, 32, 64);
    // rows were attended (their P may all have underflowed under a dominant sink)
    const bool has = any_rows;
    // the softmax denominator: the rows' sum plus an attention sink
    // (mla_v4_host.cc:469-472; LSE then covers the sink as well)
    float l = l_rows, m_fin = m_ref, o_scale = 1.0f;
    if constexpr (L::D512)
        if (p.attn_sink) {
            add_sink(l_rows, m_ref, p.attn_sink[head_q] * LOG2E, l, m_fin);
            o_scale = __builtin_amdgcn_exp2f(m_ref - m_fin);
        }
    const int64_t qrow = (int64_t)b * p.s_q + t;
    // partial results (fp32 O, LSE) in row part_row of the workspace, or the
    // final bf16 O and LSE
    const bool to_part = p.part_o != nullptr && (p.plan_items == nullptr || item_slot >= 0);
    const int64_t part_row = p.plan_items ? (int64_t)item_slot : (int64_t)split * p.B * p.s_q + qrow;
    LDS_AS float* const s_l = (LDS_AS float*)PX;      // P buffer is free now
    // one tile: P is normalised.  A list longer than the caller's bound
    // (max_kv_len / max_rows) was cut, or (656-B rows) a row's scale was
    // outside the fp16 path's range: the outputs are NaN, never a silently
    // truncated or wrong attention.
    const bool nan_out = truncated || (L::F16 && s_misc[5] != 0);
    if (hi == 0) s_l[head] = nan_out ? __builtin_nanf("") : (has ? (nchunks == 1 && ntiles == 1 ? 1.0f : o_scale / l) : 0.0f);
    if (hi == 0) {
        const float lse_v = nan_out ? __builtin_nanf("") : (m_fin + __builtin_amdgcn_logf(l)) * LN2;
        if (head_g >= p.H) {
        } else if (!to_part) {
            if (p.lse) p.lse[qrow * p.H + head_g] = has || nan_out ? lse_v : INFINITY;
        } else {
            p.part_lse[part_row * p.H + head_g] = has || nan_out ? lse_v : -FLT_MAX;
        }
    }
    __syncthreads();
    float inv[NWAVE];
#pragma unroll
    for (int h = 0; h < NWAVE; ++h) inv[h] = s_l[32 * h + r32];
    const int d0 = 128 * wave + 4 * hi;   // this lane's first output dim in block (m, g)
    if (!to_part) {
        // O through LDS, 32 heads at a time (the heads of o[4m + h]), so that
        // every global store of a wave writes one whole 1 KB head row: written
        // straight from the accumulators, each store would scatter 16-byte
        // pieces over 32 rows.  Rows are OUT_STRIDE bytes apart in the stage
        // (a 16-byte pad staggers the banks); the two tile buffers alternate.
        constexpr int OUT_STRIDE = D_VO * 2 + 16;
        static_assert(32 * OUT_STRIDE <= TILE_BYTES, "O stage fits a tile buffer");
        __bf16* const orow = p.out + (int64_t)b * p.o_sb + (int64_t)t * p.o_st;
        // per-lane stage offsets, computed here (not hoisted into the tile loop)
        const int ln = opaque_here(lane);
        const int st_w = opaque(r32 * OUT_STRIDE + 2 * d0);
        // 16-byte stores need 16-byte aligned rows; the API allows 8
        const bool o16 = ((p.o_sb | p.o_st | p.o_sh) & 7) == 0 && ((uintptr_t)p.out & 15) == 0;
#pragma unroll
        for (int h = 0; h < NWAVE; ++h) {
            const lds_ptr stg = (h & 1) ? T1 : T0;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x16& a = o[4 * m + h];
                    const f32x4 v4 = {a[4 * g] * inv[h], a[4 * g + 1] * inv[h], a[4 * g + 2] * inv[h],
                                      a[4 * g + 3] * inv[h]};
                    const bf16x4 bv = __builtin_convertvector(v4, bf16x4);
                    lds_st<u32x2>(stg + st_w + 2 * (32 * m + 8 * g), __builtin_bit_cast(u32x2, bv));
                }
            }
            __syncthreads();
            // wave w writes head rows 8w .. 8w+7 of this block, 16 bytes per lane
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int r = 8 * wave + k;
                if (hbase + 32 * h + r >= p.H) break;
                const u32x4 v = lds_ld<u32x4>(stg + r * OUT_STRIDE + 16 * ln);
                __bf16* const dst = orow + (int64_t)(hbase + 32 * h + r) * p.o_sh + 8 * ln;
                if (o16) {
                    *reinterpret_cast<u32x4*>(dst) = v;
                } else {
                    reinterpret_cast<u32x2*>(dst)[0] = u32x2{v[0], v[1]};
                    reinterpret_cast<u32x2*>(dst)[1] = u32x2{v[2], v[3]};
                }
            }
        }
    } else {
        // fp32 partials through LDS too, each wave on its own: the wave's 128
        // dims of 32 heads (16 KB; waves 0-1 in one tile buffer, 2-3 in the
        // other) leave as 512-byte row pieces, two heads per store, instead
        // of 16-byte pieces scattered over 32 rows.  A wave's LDS accesses
        // run in order, so no barrier is needed between its stage writes,
        // reads and the next head block's writes.
        constexpr int PST = D_VO + 16;        // bytes per staged head row: 128 floats + pad
        static_assert(2 * 32 * PST <= TILE_BYTES, "two waves' partial stages fit a tile buffer");
        const int ln = opaque_here(lane);
        const lds_ptr stg = (wave < 2 ? T0 : T1) + (wave & 1) * 32 * PST;
        const int st_w = opaque(r32 * PST + 16 * hi);
        const int64_t prow0 = part_row * p.H + hbase;
#pragma unroll
        for (int h = 0; h < NWAVE; ++h) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x16& a = o[4 * m + h];
                    const f32x4 v4 = {a[4 * g] * inv[h], a[4 * g + 1] * inv[h], a[4 * g + 2] * inv[h],
                                      a[4 * g + 3] * inv[h]};
                    lds_st<f32x4>(stg + st_w + 4 * (32 * m + 8 * g), v4);
                }
            }
            // lane (j, c): head row 2k + j of the block, floats 4c..4c+3 of the wave's 128
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int r = 2 * k + (ln >> 5);
                const f32x4 v = lds_ld<f32x4>(stg + r * PST + 16 * (ln & 31));
                float* op = p.part_o + (prow0 + 32 * h + r) * D_VO + 128 * wave + 4 * (ln & 31);
                if (hbase + 32 * h + r < p.H) *reinterpret_cast<f32x4*>(op) = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Narrow forward kernel (bf16 rows: 576-value rows in the top-k form or the
// CSR form with uniform splits, or the V4 prefill's 512-value rows; 656-B fp8
// rows in the same forms, dequantised to fp16 tiles): one workgroup per
// (query token, group of 32 heads, split).
// For few query tokens (low-batch decode) and small head counts: a 128-head
// workgroup per token leaves most CUs idle, or computes padding heads, while
// 32-head groups give 4x the workgroups, each with a quarter of the Q load, of
// the MFMA work per tile and of the output.  Rules as in
// dsa_mla_fwd_kernel<DSA_KV_BF16>; per tile of 32 rows:
//   QK^T     wave w = 2 hb + rb computes S^T[rows 16 rb.. x heads 16 hb..]
//            with 16x16x32 MFMAs, its 16 heads' Q in registers (each K row is
//            read by two waves, no partial scores cross the waves)
//   softmax  fixed reference (the first tile's maximum per head, taken over
//            both row halves through LDS) with one restart; 4 exponentials
//            per lane; P (bf16) goes to LDS in the PV operand layout
//   PV       split by output dims: wave w accumulates O^T[dims 128w.. x 32 heads]
// Two workgroup barriers per tile (tile landed; P written).
// grid = (B * ceil(H / 32), s_q, num_splits), block = 256.
// ---------------------------------------------------------------------------
constexpr int NARROW_HEADS = 32;
constexpr int P_BYTES = 2 * 2 * 32 * 16;      // P of a tile: [u][hi][head] x 8 bf16

__device__ __forceinline__ f32x4 mfma16_bf16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16_f16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
}

template <int NF>
__global__ void __launch_bounds__(NTHR) __attribute__((amdgpu_waves_per_eu(1, 1)))
dsa_mla_fwd_narrow_kernel(const FwdParams p_arg) {
    // row format: 576-value bf16 rows, 512-value bf16 rows (V4), or 656-B fp8
    // rows (raw tiles gathered into a ring, dequantised into fp16 tiles; the
    // NoPE MFMAs run on fp16 operands, as in dsa_mla_fwd_kernel<DSA_KV_FP8_656>)
    constexpr bool D512 = NF == DSA_KV_BF16_D512;
    constexpr bool F8 = NF == DSA_KV_FP8_656;
    static_assert(NF == DSA_KV_BF16 || D512 || F8, "narrow kernel row formats");
    // 32-deep k-steps of QK^T: 16 NoPE + 2 RoPE, or the 16 of a 512-value row
    constexpr int NKS = (D512 ? D_NOPE : D_QK) / 32;
    // bf16: a ring of three tile buffers; fp8: two fp16 tile buffers and a
    // ring of three raw slots
    __shared__ __attribute__((aligned(1024))) unsigned char s_tiles[(F8 ? 2 : 3) * TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) unsigned char s_raw[F8 ? 3 * RAW_STRIDE : 16];
    __shared__ __attribute__((aligned(16))) unsigned char s_p[P_BYTES];
    __shared__ int32_t s_rows_arr[MAX_CHUNK];
    // per-head values of the two row halves: [0] first-tile maxima, [1] one-tile
    // sums, [2] pass maxima, [3] final sums; then the references
    __shared__ float s_red_arr[4 * 2 * NARROW_HEADS + NARROW_HEADS];
    // [0..3] wave counts, [4] restart flag, [5] (fp8) a scale outside the fp16 path's range
    __shared__ int s_misc_arr[NWAVE + 2];
    const lds_ptr TB = (lds_ptr)s_tiles;
    const lds_ptr PX = (lds_ptr)s_p;
    LDS_AS int32_t* const s_rows = (LDS_AS int32_t*)s_rows_arr;
    LDS_AS float* const s_red = (LDS_AS float*)s_red_arr;
    LDS_AS int* const s_misc = (LDS_AS int*)s_misc_arr;
    // The arguments the prologue reads, copied into registers in one batch
    // (opaque copies, which the compiler cannot reload where they are used):
    // left to the compiler, the scalar loads of the argument block form a
    // chain across the branches below, one memory round trip each.
    FwdParams p = p_arg;
    unsigned grid_x = gridDim.x, grid_z = gridDim.z;
    uintptr_t a_q = (uintptr_t)p.q, a_bt = (uintptr_t)p.block_table, a_sl = (uintptr_t)p.seq_lens,
              a_ix = (uintptr_t)p.indices, a_ip = (uintptr_t)p.kv_indptr, a_ki = (uintptr_t)p.kv_indices;
    uintptr_t a_o = (uintptr_t)p.out, a_lse = (uintptr_t)p.lse, a_po = (uintptr_t)p.part_o, a_pl = (uintptr_t)p.part_lse;
    asm volatile(""
                 : "+s"(grid_x), "+s"(grid_z), "+s"(a_q), "+s"(a_bt), "+s"(a_sl), "+s"(a_ix), "+s"(a_ip), "+s"(a_ki),
                   "+s"(p.q_sb), "+s"(p.q_st), "+s"(p.q_sh), "+s"(p.kv_total_rows), "+s"(p.kv_batch_stride),
                   "+s"(p.bt_stride), "+s"(p.block_size), "+s"(p.bs_shift), "+s"(p.seq_len_default), "+s"(p.idx_sb),
                   "+s"(p.idx_st), "+s"(p.s_q), "+s"(p.topk), "+s"(p.chunk), "+s"(p.H), "+s"(p.hgroups),
                   "+s"(p.causal), "+s"(p.causal_offset), "+s"(p.reverse), "+s"(a_o), "+s"(p.o_sb), "+s"(p.o_st),
                   "+s"(p.o_sh), "+s"(a_lse), "+s"(a_po), "+s"(a_pl));
    if constexpr (D512) {
        uintptr_t a_np = (uintptr_t)p.ind_pre, a_xp = (uintptr_t)p.idx_pre, a_ne = (uintptr_t)p.ind_ext,
                  a_xe = (uintptr_t)p.idx_ext, a_sk = (uintptr_t)p.attn_sink;
        asm volatile("" : "+s"(a_np), "+s"(a_xp), "+s"(a_ne), "+s"(a_xe), "+s"(a_sk), "+s"(p.kv2_rows));
        p.ind_pre = gptr<const int32_t>(a_np);
        p.idx_pre = gptr<const int32_t>(a_xp);
        p.ind_ext = gptr<const int32_t>(a_ne);
        p.idx_ext = gptr<const int32_t>(a_xe);
        p.attn_sink = gptr<const float>(a_sk);
    }
    p.out = gptr<__bf16>(a_o);
    p.lse = gptr<float>(a_lse);
    p.part_o = gptr<float>(a_po);
    p.part_lse = gptr<float>(a_pl);
    p.q = gptr<const __bf16>(a_q);
    p.block_table = gptr<const int32_t>(a_bt);
    p.seq_lens = gptr<const int32_t>(a_sl);
    p.indices = gptr<const int32_t>(a_ix);
    p.kv_indptr = gptr<const int32_t>(a_ip);
    p.kv_indices = gptr<const int32_t>(a_ki);

    // blockIdx.x = query token * hgroups + head group
    const int gx = (int)blockIdx.x / p.hgroups;
    const int hbase = NARROW_HEADS * ((int)blockIdx.x % p.hgroups);
    const int b = p.reverse ? (int)(grid_x / p.hgroups) - 1 - gx : gx, t = blockIdx.y;
    const int split = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = wave & 1, hb = wave >> 1;      // QK^T: row half, head half
    const int c16 = lane & 15, g4 = lane >> 4;    // 16x16 operand lanes
    const int hi = lane >> 5, r32 = lane & 31;    // PV and epilogue lanes: head r32
    const int hq = 16 * hb + c16;                 // this lane's head in QK^T and the softmax
    // heads past H are computed on a copy of head H-1 and never stored
    const int head_g = hbase + r32;
    if (tid == 0) {
        s_misc[NWAVE] = 0;
        s_misc[NWAVE + 1] = 0;
    }

    // ---- this split's entries, by the rules of dsa_mla_fwd_kernel.  Top-k
    // form: logical positions through the block table, bounded by seq_len and
    // the causal rule.  CSR form (uniform splits): physical rows
    // kv_indices[kv_indptr[b] + k], k below the count-based MTP bound.  V4
    // prefill: the prefix rows of kv, then the extend rows of kv2 (POOL2),
    // at most max_rows of them (a longer list is cut, NaN), the splits taking
    // whole tiles (opus_attn/dsa_v4/common/mla_prefill_split.h:34-44) ----
    int k0 = split * p.chunk;
    int k1;
    const int32_t* idx;
    bool truncated = false;
    int64_t v4_np = 0, v4_eb = 0;
    if constexpr (D512) {
        const int64_t pb = sload(p.ind_pre + b);
        v4_np = max((int64_t)sload(p.ind_pre + b + 1) - pb, (int64_t)0);
        v4_eb = sload(p.ind_ext + b);
        const int64_t ne = max((int64_t)sload(p.ind_ext + b + 1) - v4_eb, (int64_t)0);
        const int64_t n_b = min(v4_np + ne, (int64_t)p.topk);
        truncated = v4_np + ne > p.topk;
        const int64_t per = (n_b + grid_z - 1) / grid_z;
        const int64_t cb = (per + TILE - 1) / TILE * TILE;
        k0 = (int)min((int64_t)split * cb, n_b);
        k1 = (int)min((int64_t)k0 + cb, n_b);
        idx = p.idx_pre + pb;
    } else if (p.kv_indptr) {
        const int64_t kb = sload(p.kv_indptr + b);
        const int64_t count = (int64_t)sload(p.kv_indptr + b + 1) - kb - (p.s_q - 1 - t);
        k1 = (int)min((int64_t)k0 + p.chunk, count);
        // a list longer than the splits cover (max_kv_len) is cut: NaN
        truncated = count > (int64_t)grid_z * p.chunk;
        idx = p.kv_indices + kb;
    } else {
        k1 = (int)min((int64_t)k0 + p.chunk, (int64_t)p.topk);
        idx = p.indices + (int64_t)b * p.idx_sb + (int64_t)t * p.idx_st;
    }
    const int nchunks = k1 > k0 ? (k1 - k0 + MAX_CHUNK - 1) / MAX_CHUNK : 1;
    constexpr int PER_T = MAX_CHUNK / NTHR;       // entries per thread and chunk
    // the entries of chunk c (-1 past the split's end); V4: entry k is an
    // extend entry from k = v4_np on
    auto load_entries = [&](int c, int32_t (&jv)[PER_T]) {
        const int kc0 = k0 + c * MAX_CHUNK;
        const int kc1 = min(kc0 + MAX_CHUNK, k1);
#pragma unroll
        for (int e = 0; e < PER_T; ++e) {
            const int k = kc0 + tid * PER_T + e;
            if (D512 && k >= v4_np) jv[e] = k < kc1 ? p.idx_ext[v4_eb + (k - v4_np)] : -1;
            else jv[e] = k < kc1 ? idx[k] : -1;
        }
    };
    // Chunk 0's entries are loaded before Q: vmcnt counts in order, so the wait
    // for them does not wait for the Q loads as well.
    int32_t jv0[PER_T], ent0[PER_T];
    load_entries(0, jv0);
    // top-k form: the bound on positions, from seq_len and the causal rule
    // (a scalar load, in flight with the entries)
    int64_t jmax = 0;
    const bool topk_form = !D512 && !p.kv_indptr;
    if (topk_form) {
        const int64_t Lq = p.seq_lens ? (int64_t)sload(p.seq_lens + b) : p.seq_len_default;
        jmax = Lq;
        if (p.causal == 1) jmax = min(Lq, Lq - p.s_q + t + 1);
        else if (p.causal == 2) jmax = min(Lq, (int64_t)b + p.causal_offset + 1);
    }
    // a paged top-k list's block-table reads for those entries go out before
    // Q as well: waiting for them then does not wait for Q
    const bool topk_paged = topk_form && p.block_table;
    if (topk_paged) topk_ents(p, b, jmax, jv0, ent0);

    // ---- Q fragments (B operand of S^T = K Q^T): head hq, dims 32 ks + 8 g4 .. +7 ----
    u32x4 qf[NKS];
    {
        const __bf16* qp = p.q + (int64_t)b * p.q_sb + (int64_t)t * p.q_st +
                           (int64_t)min(hbase + hq, p.H - 1) * p.q_sh + 8 * g4;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qp + 32 * ks);
    }
    // the softmax scale (log2 units) of this lane's head hq
    float c_s = p.scale_log2;
    // fp8 rows, once Q has landed: its NoPE part to fp16 for the fp16 MFMAs.
    // A head with |q| >= 2^15 would leave fp16's range: the whole head (NoPE
    // and RoPE) is scaled by 2^-k, bringing its largest NoPE value below
    // 2^15, and c_s by 2^k, so the scaled scores are the same; both are exact,
    // and k = 0 for every |q| < 2^15 (as in dsa_mla_fwd_kernel).  A head's
    // dims are spread over the four lanes g4 of column c16.
    auto convert_q = [&]() {
        if constexpr (F8) {
            typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
            u16x2 amax = {0, 0};
#pragma unroll
            for (int ks = 0; ks < KS_NOPE / 2; ++ks)
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    amax = __builtin_elementwise_max(amax, __builtin_bit_cast(u16x2, qf[ks][w] & 0x7FFF7FFFu));
            // biased exponent of the head's largest |q| (bf16 bits >> 7)
            int eb = max((int)amax[0], (int)amax[1]) >> 7;
            eb = max(eb, __shfl_xor(eb, 16, 64));
            eb = max(eb, __shfl_xor(eb, 32, 64));
            const int k = max(eb - 141, 0);                   // 141 = 127 + 14
            const float s = __uint_as_float((unsigned)(127 - k) << 23);
            c_s = p.scale_log2 * __uint_as_float((unsigned)(127 + k) << 23);
#pragma unroll
            for (int ks = 0; ks < KS_NOPE / 2; ++ks)
#pragma unroll
                for (int w = 0; w < 4; ++w) qf[ks][w] = bf16x2_to_f16x2(qf[ks][w], s);
#pragma unroll
            for (int ks = KS_NOPE / 2; ks < NKS; ++ks)
#pragma unroll
                for (int w = 0; w < 4; ++w) qf[ks][w] = bf16x2_scale(qf[ks][w], s);
        }
    };

    // entries of chunk c -> the compacted row list, the last tile padded with
    // copies of the first valid row (ends with a barrier)
    int n_valid = 0, ntiles = 0;
    bool any_rows = false;
    auto resolve_chunk = [&](int c, bool preloaded) {
        int32_t rows_local[PER_T];
        int cnt = 0;
        {
            int32_t jv[PER_T];
            if (preloaded) {
#pragma unroll
                for (int e = 0; e < PER_T; ++e) jv[e] = jv0[e];
            } else {
                load_entries(c, jv);
            }
            if constexpr (D512) {
                const int kc0 = k0 + c * MAX_CHUNK;
#pragma unroll
                for (int e = 0; e < PER_T; ++e)
                    rows_local[e] = kc0 + tid * PER_T + e >= v4_np ? dsa_rows::v4_extend_row(jv[e], p.kv2_rows)
                                                                   : dsa_rows::v4_prefix_row(jv[e], p.kv_total_rows);
            } else if (p.kv_indptr) {
#pragma unroll
                for (int e = 0; e < PER_T; ++e) rows_local[e] = dsa_rows::csr_row(jv[e], p.kv_total_rows);
            } else {
                int32_t ent[PER_T];
                if (preloaded && topk_paged) {
#pragma unroll
                    for (int e = 0; e < PER_T; ++e) ent[e] = ent0[e];
                } else {
                    topk_ents(p, b, jmax, jv, ent);
                }
                topk_rows_of(p, b, jv, ent, rows_local);
            }
#pragma unroll
            for (int e = 0; e < PER_T; ++e) cnt += rows_local[e] >= 0 ? 1 : 0;
        }
        const int incl = wave_incl_sum16(cnt);
        // (the barrier also ends every wave's use of the previous chunk's row
        // list, tile buffers and P)
        if (lane == 63) s_misc[wave] = incl;
        __syncthreads();
        int wbase = 0, nv = 0;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) {
            const int s = s_misc[w];
            wbase += w < wave ? s : 0;
            nv += s;
        }
        {
            int pos = wbase + incl - cnt;
#pragma unroll
            for (int e = 0; e < PER_T; ++e)
                if (rows_local[e] >= 0) s_rows[pos++] = rows_local[e];
        }
        // (wave-uniform: every wave summed the same counts)
        n_valid = __builtin_amdgcn_readfirstlane(nv);
        ntiles = (n_valid + TILE - 1) / TILE;
        any_rows = any_rows || nv > 0;
        __syncthreads();
        if (tid < TILE && nv > 0 && nv + tid < ntiles * TILE) s_rows[nv + tid] = s_rows[0];
        __syncthreads();
    };

    // ---- gather: wave w loads NoPE rows 8w..8w+7 (one 1 KB LDS-DMA load per
    // row) and the RoPE blocks of those rows (one load; none for 512-value
    // rows, whose row ids name their pool); tile layout and swizzles as in
    // dsa_mla_fwd_kernel ----
    struct GatherRows {
        int32_t r[TILE / NWAVE];   // this wave's rows (uniform)
        int32_t rope;              // row of this lane's RoPE chunk
    };
    auto slot = [&](int s) -> lds_ptr { return TB + s * TILE_BYTES; };
    // 656-B rows: the raw tile's 1312 16-byte chunks (rows back to back) are 21
    // loads, wave w taking loads w, w+4, ... (6 for wave 0, 5 for the others);
    // lane chunk c16 = 64 k + lane of load k lies in row c16 / 41 of the tile,
    // at chunk c16 % 41.  Per lane and load: bits 0..15 the byte offset of the
    // row's id in the row list (row clamped to 31: the last load's spare lanes
    // read chunks of row 31 into the slot's padding), bits 16..31 the chunk's
    // byte offset in the row (as in dsa_mla_fwd_kernel).
    const lds_ptr RAW = (lds_ptr)s_raw;
    const int my_loads = F8 ? (wave < FP8_LOADS - NWAVE * (FP8_LPW - 1) ? FP8_LPW : FP8_LPW - 1) : 0;
    uint32_t f_rc[FP8_LPW] = {};
    if constexpr (F8) {
#pragma unroll
        for (int i = 0; i < FP8_LPW; ++i) {
            const unsigned c16 = 64 * (wave + NWAVE * i) + lane;
            const unsigned rt = c16 / 41u;
            f_rc[i] = 4u * (rt < TILE - 1 ? rt : TILE - 1) | (16u * (c16 - 41u * rt)) << 16;
        }
    }
    auto load_rows = [&](int ti) -> GatherRows {
        const LDS_AS int32_t* rows = s_rows + ti * TILE;
        GatherRows g;
        if constexpr (F8) {
            // (an opaque copy: the unpacked halves would be hoisted out of the loop)
#pragma unroll
            for (int i = 0; i < FP8_LPW; ++i)
                g.r[i] = lds_ld<int32_t>((lds_cptr)rows + ((unsigned)opaque((int)f_rc[i]) & 0xFFFFu));
            g.rope = 0;
            return g;
        }
        const u32x4 ra = lds_ld<u32x4>((lds_cptr)(rows + 8 * wave));
        const u32x4 rv = lds_ld<u32x4>((lds_cptr)(rows + 8 * wave + 4));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            g.r[i] = __builtin_amdgcn_readfirstlane((int)ra[i]);
            g.r[4 + i] = __builtin_amdgcn_readfirstlane((int)rv[i]);
        }
        g.rope = rows[8 * wave + (opaque(lane) >> 3)];
        return g;
    };
    auto issue_rows = [&](const GatherRows& g, lds_ptr tb) {
        const int ln = opaque(lane);
        if constexpr (F8) {
            // tb: the raw slot
#pragma unroll
            for (int i = 0; i < FP8_LPW; ++i)
                if (i < my_loads) {
                    const uint64_t row = (uint32_t)g.r[i];
                    lds_dma16(p.kv + (row * (uint32_t)p.row_bytes + ((unsigned)opaque((int)f_rc[i]) >> 16)),
                              tb + 1024 * (wave + NWAVE * i));
                }
            return;
        }
#pragma unroll
        for (int i = 0; i < TILE / NWAVE; ++i) {
            const int r = 8 * wave + i;
            const int32_t id = __builtin_amdgcn_readfirstlane(g.r[i]);
            const unsigned char* base;
            if constexpr (D512)
                base = (dsa_rows::row_in_pool2(id) ? p.kv2 : p.kv) + (int64_t)dsa_rows::row_index(id) * p.row_bytes;
            else
                base = p.kv + (int64_t)id * p.row_bytes;
            lds_dma16_s(base, 16u * (unsigned)(ln ^ nope_sw(r)), tb + r * NOPE_STRIDE);
        }
        if constexpr (!D512) {
            const int r = 8 * wave + (ln >> 3);
            lds_dma16(p.kv + (int64_t)g.rope * p.row_bytes + 2 * D_NOPE + 16 * ((ln & 7) ^ rope_sw(r)),
                      tb + ROPE_OFF + 8 * wave * 128);
        }
    };
    constexpr int LPW = TILE / NWAVE + (D512 ? 0 : 1);     // loads per wave per tile (bf16 rows)
    // fp8: wait until this wave's loads of all but the newest `keep` tiles landed
    auto wait_keep = [&](int keep) {
        if (keep <= 0) wait_vm<0>();
        else if (keep == 1) {
            if (my_loads == FP8_LPW) wait_vm<FP8_LPW>();
            else wait_vm<FP8_LPW - 1>();
        } else {
            if (my_loads == FP8_LPW) wait_vm<2 * FP8_LPW>();
            else wait_vm<2 * (FP8_LPW - 1)>();
        }
    };
    // fp8: raw slot rb -> fp16 tile buffer tb, cooperatively.  Pieces 0..7:
    // wave w converts row w + 4j, lane l the NoPE codes 8l..8l+7 of scale
    // group l/16 (fp16 = fp16(code * 2^e) * fp16(mantissa) for scale =
    // mantissa * 2^e); piece 8: the RoPE values, one 16-byte chunk per thread,
    // copied as bf16.  A scale at or above FP8_SCALE_LIMIT_BITS sets range_bad
    // (the outputs then become NaN).  All loads are issued before any store.
    bool range_bad = false;
    auto dequant_tile = [&](lds_cptr rb, lds_ptr tb) {
        const int ln = opaque(lane);
        u32x2 codes[TILE / NWAVE];
        unsigned sbits[TILE / NWAVE];
#pragma unroll
        for (int j = 0; j < TILE / NWAVE; ++j) {
            const lds_cptr rr = rb + (wave + NWAVE * j) * FP8_ROW;
            codes[j] = lds_ld<u32x2>(rr + 8 * ln);
            sbits[j] = lds_ld<unsigned>(rr + FP8_SCALE_OFF + 4 * (ln >> 4));
        }
        const int t8 = opaque(tid);
        const u32x4 rope = lds_ld<u32x4>(rb + (t8 >> 3) * FP8_ROW + FP8_ROPE_OFF + 16 * (t8 & 7));
        bool bad = false;
#pragma unroll
        for (int j = 0; j < TILE / NWAVE; ++j) {
            const int r = wave + NWAVE * j;
            const float sc = __uint_as_float(sbits[j]);
            bad |= sbits[j] >= FP8_SCALE_LIMIT_BITS;
            const _Float16 m16 = (_Float16)__uint_as_float((sbits[j] & 0x007FFFFFu) | 0x3F800000u);
            const f16x2 mm = {m16, m16};
            const f16x2 h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)codes[j][0], sc, false) * mm;
            const f16x2 h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)codes[j][0], sc, true) * mm;
            const f16x2 h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)codes[j][1], sc, false) * mm;
            const f16x2 h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)codes[j][1], sc, true) * mm;
            const u32x4 out = {__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1),
                               __builtin_bit_cast(unsigned, h2), __builtin_bit_cast(unsigned, h3)};
            lds_st<u32x4>(tb + r * NOPE_STRIDE + 16 * (ln ^ nope_sw(r)), out);
        }
        const int rr8 = t8 >> 3, cc8 = t8 & 7;
        lds_st<u32x4>(tb + ROPE_OFF + 128 * rr8 + 16 * (cc8 ^ rope_sw(rr8)), rope);
        range_bad |= bad;
    };

    // ---- S^T[16 rows x 16 heads] = K Q^T (A operand: row 16 rb + c16, dims
    // 32 ks + 8 g4 .. +7, i.e. chunk 4 ks + g4 at its swizzled position) ----
    auto qk16 = [&](lds_cptr kt) -> f32x4 {
        const int ln = opaque(lane);
        const int row = 16 * rb + (ln & 15), lg = ln >> 4;
        const lds_cptr kn = kt + row * NOPE_STRIDE + 16 * (lg ^ nope_sw(row));
        const lds_cptr kr = kt + ROPE_OFF + 128 * row;
        const int rsw = rope_sw(row);
        auto k_addr = [&](int ks) -> lds_cptr {
            return ks < KS_NOPE / 2 ? kn + 64 * ks : kr + 16 * ((4 * (ks - KS_NOPE / 2) + lg) ^ rsw);
        };
        constexpr int KPF = 6;
        u32x4 kb[KPF];
#pragma unroll
        for (int i = 0; i < KPF; ++i) kb[i] = lds_ld<u32x4>(k_addr(i));
        // two accumulator chains (a single 16x16x32 chain is latency-bound)
        f32x4 acc[2] = {};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            __builtin_amdgcn_sched_barrier(0);
            // (fp8 rows: the NoPE k-steps on fp16 operands, RoPE on bf16)
            if (F8 && ks < KS_NOPE / 2) acc[ks & 1] = mfma16_f16(kb[ks % KPF], qf[ks], acc[ks & 1]);
            else acc[ks & 1] = mfma16_bf16(kb[ks % KPF], qf[ks], acc[ks & 1]);
            if (ks + KPF < NKS) kb[ks % KPF] = lds_ld<u32x4>(k_addr(ks + KPF));
        }
        __builtin_amdgcn_sched_barrier(0);
        return acc[0] + acc[1];
    };

    // softmax state of head hq over this wave's rows: lane (g4, c16), value i
    // of the 16x16 tile is row 16 rb + 4 g4 + i of the tile
    float m_ref = 0.0f, l_lane = 0.0f, s_max = -INFINITY;
    bool first_tile = true;
    // per head over the wave's 16 rows (the 4 lanes g4 of head c16)
    auto red4_max = [&](float v) {
        v = fmaxf(v, __shfl_xor(v, 16, 64));
        return fmaxf(v, __shfl_xor(v, 32, 64));
    };
    auto red4_sum = [&](float v) {
        v += __shfl_xor(v, 16, 64);
        return v + __shfl_xor(v, 32, 64);
    };
    // per-head value of both row halves through LDS slot k (a barrier between)
    auto put_half = [&](int k, float v) {
        if (g4 == 0) s_red[(2 * k + rb) * NARROW_HEADS + hq] = v;
    };
    auto get_max = [&](int k) { return fmaxf(s_red[2 * k * NARROW_HEADS + hq], s_red[(2 * k + 1) * NARROW_HEADS + hq]); };

    // O^T accumulators: dims 128 wave + 32 m + (0..31) of the 32 heads: o[m]
    f32x16 o[4];
    // Chunk 0 of pass 0, from the preloaded entries, outside the pass loop: a
    // call inside it shared its code with the calls that load their entries
    // just before use, and the compiler's wait for those (vmcnt(0)) then
    // drained the Q loads on this path too.
    resolve_chunk(0, true);
    for (int pass = 0;; ++pass) {
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = f32x16{};
        l_lane = 0.0f;
        s_max = -INFINITY;
        first_tile = pass == 0;
        for (int c = 0; c < nchunks; ++c) {
            // a one-chunk list keeps its row list for the second pass
            if ((pass == 0 && c > 0) || (pass > 0 && nchunks > 1)) resolve_chunk(c, false);
            // The index loads have completed (the row list is built); Q's may
            // still be in flight: they are older than the gathers, so the tile
            // loop's in-order waits for a tile's gathers cover them too.
            // bf16 rows: tiles 0 and 1 go out before the loop, tile it+2 in
            // iteration it, into ring slot (it+2) % 3.  fp8 rows: raw tiles 0..2
            // before the loop, raw tile it+3 in iteration it into raw slot it % 3
            // (dequantised in iteration it-1); tile j is dequantised into fp16
            // buffer j % 2 after the PV of tile j-1.
            constexpr int NPRE = F8 ? 3 : 2;
            auto ring = [&](int s) -> lds_ptr { return F8 ? RAW + s * RAW_STRIDE : slot(s); };
#pragma unroll
            for (int s0 = 0; s0 < NPRE; ++s0)
                if (s0 < ntiles) issue_rows(load_rows(s0), ring(s0));
            GatherRows gnext;
            if (NPRE < ntiles) gnext = load_rows(NPRE);
            if constexpr (F8) {
                if (pass == 0 && c == 0) convert_q();
                if (ntiles > 0) {
                    wait_keep(min(ntiles, NPRE) - 1);    // raw tile 0 landed
                    tile_barrier();
                    dequant_tile(RAW, TB);
                }
            }
            for (int it = 0; it < ntiles; ++it) {
                // bf16: tile it landed (tile it+1 may be in flight); fp8: raw
                // tile it+1 landed (it+2 may be in flight).  After the barrier
                // every wave is done with tile it-1 (bf16: its slot receives
                // tile it+2; fp8: its fp16 buffer receives tile it+1) and with
                // its P; fp8: tile it's fp16 buffer is complete.
                if constexpr (F8) {
                    wait_keep(it + 2 < ntiles ? 1 : 0);
                } else {
                    if (it + 1 < ntiles) wait_vm<LPW>();
                    else wait_vm<0>();
                }
                tile_barrier();
                const lds_ptr kt = F8 ? TB + (it & 1) * TILE_BYTES : slot(it % 3);
                __builtin_amdgcn_sched_barrier(0);
                if (it + NPRE < ntiles) issue_rows(gnext, ring((it + NPRE) % 3));
                __builtin_amdgcn_sched_barrier(0);
                f32x4 s = qk16(kt);
                // ---- V^T operands of PV (transposed reads): 16-lane group g16
                // reads rows R..R+3 (lane 4rr+pp: row R+rr, dims d0+4pp..+3) with
                // R = 16u + 4hi and R + 8 ----
                const int vln = opaque(lane);
                const int vhi = vln >> 5;
                const int g16 = vln >> 4, i16 = vln & 15, vrr = i16 >> 2, vpp = i16 & 3;
                const int vx = 2 * (g16 & 1) + (vpp >> 1);
                const lds_cptr v_a = kt + (4 * vhi + vrr) * NOPE_STRIDE + 16 * (vx ^ vhi) + 8 * (vpp & 1) + 256 * wave;
                const lds_cptr v_b =
                    kt + (4 * vhi + vrr + 8) * NOPE_STRIDE + 16 * (vx ^ (vhi + 2)) + 8 * (vpp & 1) + 256 * wave;
                auto v_frag = [&](int u, int m) -> u32x4 {
                    const s16x4 va = lds_read_tr16(v_a + 16 * u * NOPE_STRIDE + 64 * m);
                    const s16x4 vb = lds_read_tr16(v_b + 16 * u * NOPE_STRIDE + 64 * m);
                    return __builtin_bit_cast(u32x4, __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7));
                };
                const int rows_left = n_valid - it * TILE;
                const int row0 = 16 * rb + 4 * g4;
                if (first_tile) {
                    // the reference: the largest score of the list's first tile
                    float mx = -INFINITY;
#pragma unroll
                    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, row0 + i < rows_left ? s[i] : -INFINITY);
                    put_half(0, red4_max(mx));
                    tile_barrier();
                    m_ref = get_max(0) * c_s;
                    first_tile = false;
                }
                if (rows_left < TILE) {
                    asm volatile("");
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[i] = row0 + i < rows_left ? s[i] : -INFINITY;
                }
                s_max = fmaxf(s_max, fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
                if (nchunks == 1 && ntiles == 1) {
                    // single-tile list: the exact sum folded into the reference,
                    // so that P is normalised when it is rounded
                    // (opus_attn/dsa_v32/common/host.cc:448-451)
                    float lt = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) lt += __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c_s, -m_ref));
                    put_half(1, red4_sum(lt));
                    tile_barrier();
                    float l1 = s_red[2 * NARROW_HEADS + hq] + s_red[3 * NARROW_HEADS + hq], m_fold = m_ref;
                    // (an attention sink joins the sum: mla_v4_host.cc:469-472)
                    if (D512 && p.attn_sink)
                        add_sink(l1, m_ref, p.attn_sink[min(hbase + hq, p.H - 1)] * LOG2E, l1, m_fold);
                    m_ref = m_fold + __builtin_amdgcn_logf(l1);
                }
                f32x4 e;
#pragma unroll
                for (int i = 0; i < 4; ++i) e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c_s, -m_ref));
                l_lane += (e[0] + e[1]) + (e[2] + e[3]);
                // P of rows 16 rb + 4 g4 + i: PV k-step u = rb, lane half g4 & 1,
                // positions 4 (g4 >> 1) + i (the rows the V reads pair with them)
                u32x2 pw;
                if constexpr (F8) {
                    // fp16 P for the fp16 PV MFMAs (finite below 2^16: TAU = 15)
                    const f16x2 p01 = {(_Float16)e[0], (_Float16)e[1]}, p23 = {(_Float16)e[2], (_Float16)e[3]};
                    pw = u32x2{__builtin_bit_cast(unsigned, p01), __builtin_bit_cast(unsigned, p23)};
                } else {
                    pw = __builtin_bit_cast(u32x2, __builtin_convertvector(e, bf16x4));
                }
                lds_st<u32x2>(PX + ((2 * rb + (g4 & 1)) * NARROW_HEADS + hq) * 16 + 8 * (g4 >> 1), pw);
                tile_barrier();
                // ---- O^T[128 dims of this wave x 32 heads] += V^T P^T ----
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const u32x4 pb = lds_ld<u32x4>(PX + ((2 * u + vhi) * NARROW_HEADS + (vln & 31)) * 16);
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        if constexpr (F8) o[m] = mfma_f16(v_frag(u, m), pb, o[m]);
                        else o[m] = mfma_bf16(v_frag(u, m), pb, o[m]);
                    }
                }
                // fp8: tile it+1 (landed) into the other fp16 buffer
                if constexpr (F8)
                    if (it + 1 < ntiles)
                        dequant_tile(RAW + ((it + 1) % 3) * RAW_STRIDE, TB + ((it + 1) & 1) * TILE_BYTES);
                if (it + NPRE + 1 < ntiles) gnext = load_rows(it + NPRE + 1);
            }
            // drain in-flight gathers before the slots can be reused or left
            wait_vm<0>();
        }
        // per head: the largest score of the pass over both row halves (log2
        // units); NaN compares false.  A head past the reference by more than
        // TAU restarts the workgroup once, with the exact maximum.
        put_half(2, red4_max(s_max));
        // (the barrier also ends every wave's use of the tile buffers: a
        // restart refills them, the epilogue stages O in them)
        tile_barrier();
        const float top = get_max(2) * c_s;
        if (pass == 0 && __builtin_amdgcn_ballot_w64(top - m_ref > Lay<F8 ? DSA_KV_FP8_656 : DSA_KV_BF16>::TAU) != 0 &&
            lane == 0)
            s_misc[NWAVE] = 1;
        tile_barrier();
        if (pass != 0 || s_misc[NWAVE] == 0) break;
        m_ref = fmaxf(m_ref, top);
    }

    // ---- epilogue: O / l and LSE, final (bf16) or a split's partial (fp32) ----
    // the sums and references per head, from the QK^T lanes to the PV lanes (head r32)
    put_half(3, red4_sum(l_lane));
    if (rb == 0 && g4 == 0) s_red[8 * NARROW_HEADS + hq] = m_ref;
    if (F8 && range_bad) s_misc[NWAVE + 1] = 1;
    tile_barrier();
    // A list cut short, or (fp8 rows) a scale outside the fp16 path's range:
    // NaN outputs, never a silently truncated or wrong attention.
    const bool nan_out = truncated || (F8 && s_misc[NWAVE + 1] != 0);
    const float l_rows = s_red[6 * NARROW_HEADS + r32] + s_red[7 * NARROW_HEADS + r32];
    const float m_head = s_red[8 * NARROW_HEADS + r32];
    const bool has = any_rows;
    // the softmax denominator: the rows' sum plus an attention sink
    // (mla_v4_host.cc:469-472; LSE then covers the sink as well)
    float l = l_rows, m_fin = m_head, o_scale = 1.0f;
    if constexpr (D512)
        if (p.attn_sink) {
            add_sink(l_rows, m_head, p.attn_sink[min(head_g, p.H - 1)] * LOG2E, l, m_fin);
            o_scale = __builtin_amdgcn_exp2f(m_head - m_fin);
        }
    const float inv =
        nan_out ? __builtin_nanf("") : (has ? (nchunks == 1 && ntiles == 1 ? 1.0f : o_scale / l) : 0.0f);
    const int64_t qrow = (int64_t)b * p.s_q + t;
    const bool to_part = p.part_o != nullptr;
    const int64_t part_row = (int64_t)split * p.B * p.s_q + qrow;
    if (wave == 0 && hi == 0 && head_g < p.H) {
        const float lse_v = nan_out ? __builtin_nanf("") : (m_fin + __builtin_amdgcn_logf(l)) * LN2;
        if (!to_part) {
            if (p.lse) p.lse[qrow * p.H + head_g] = has || nan_out ? lse_v : INFINITY;
        } else {
            p.part_lse[part_row * p.H + head_g] = has || nan_out ? lse_v : -FLT_MAX;
        }
    }
    // lane (hi, r32), reg 4g + i of o[m]: dim 128 wave + 32 m + 8 g + 4 hi + i of head r32.
    // Staged through LDS (each wave its own region) so that the global stores
    // write whole row pieces of the wave's 128 dims.
    const int ln = opaque(lane);
    if (!to_part) {
        constexpr int OST = 2 * 128 + 16;               // staged head row: 128 bf16 + pad
        static_assert(NWAVE * 32 * OST <= TILE_BYTES, "O stage fits a tile buffer");
        const lds_ptr stg = TB + wave * 32 * OST;
        const int st_w = opaque(r32 * OST + 8 * hi);
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v4 = {o[m][4 * g] * inv, o[m][4 * g + 1] * inv, o[m][4 * g + 2] * inv,
                                  o[m][4 * g + 3] * inv};
                lds_st<u32x2>(stg + st_w + 2 * (32 * m + 8 * g), __builtin_bit_cast(u32x2, __builtin_convertvector(v4, bf16x4)));
            }
        __bf16* const orow = p.out + (int64_t)b * p.o_sb + (int64_t)t * p.o_st;
        const bool o16 = ((p.o_sb | p.o_st | p.o_sh) & 7) == 0 && ((uintptr_t)p.out & 15) == 0;
        // lane (k, c): head row 4k + c / 16 of the group, dims 8 (c % 16) .. +7 of the wave's 128
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int r = 4 * k + (ln >> 4);
            if (hbase + r >= p.H) break;
            const u32x4 v = lds_ld<u32x4>(stg + r * OST + 16 * (ln & 15));
            __bf16* const dst = orow + (int64_t)(hbase + r) * p.o_sh + 128 * wave + 8 * (ln & 15);
            if (o16) {
                *reinterpret_cast<u32x4*>(dst) = v;
            } else {
                reinterpret_cast<u32x2*>(dst)[0] = u32x2{v[0], v[1]};
                reinterpret_cast<u32x2*>(dst)[1] = u32x2{v[2], v[3]};
            }
        }
    } else {
        constexpr int PST = 4 * 128 + 16;               // staged head row: 128 floats + pad
        static_assert(2 * 32 * PST <= TILE_BYTES, "two waves' partial stages fit a tile buffer");
        const lds_ptr stg = TB + (wave >> 1) * TILE_BYTES + (wave & 1) * 32 * PST;
        const int st_w = opaque(r32 * PST + 16 * hi);
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v4 = {o[m][4 * g] * inv, o[m][4 * g + 1] * inv, o[m][4 * g + 2] * inv,
                                  o[m][4 * g + 3] * inv};
                lds_st<f32x4>(stg + st_w + 4 * (32 * m + 8 * g), v4);
            }
        const int64_t prow0 = part_row * p.H + hbase;
        // lane (j, c): head row 2k + j of the group, floats 4c..4c+3 of the wave's 128
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int r = 2 * k + (ln >> 5);
            const f32x4 v = lds_ld<f32x4>(stg + r * PST + 16 * (ln & 31));
            if (hbase + r < p.H)
                *reinterpret_cast<f32x4*>(p.part_o + (prow0 + r) * D_VO + 128 * wave + 4 * (ln & 31)) = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Split combine: one wave per (row, head); lane holds 8 of the 512 outputs.
// Math of mla_reduce (opus_attn/dsa_v32/common/mla_reduce.hpp:6-156):
// m = max lse_i, w_i = exp(lse_i - m) (0 for an empty split),
// O = sum w_i O_i / sum w_i, LSE = m + ln sum w_i (+inf when all are empty).
// Uniform splits: grid = (rows, min(H, 65535)), block = 64.
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// CSR work plan: one workgroup of 256 threads, on the device (the host cannot
// read the lists).  Query row q = b * s_q + t attends
// L_q = kv_indptr[b+1] - kv_indptr[b] - (s_q - 1 - t) entries (count-based
// MTP causality).  The plan cuts the lists into work items of at most
// `chunk` entries (a multiple of the tile, >= PLAN_MIN_CHUNK): below
// PLAN_TARGET rows the smallest chunk whose items fit one round of
// PLAN_TARGET workgroups, from PLAN_TARGET rows on total / PLAN_TARGET (a row
// longer than that splits, an average one does not).  However the lengths
// are spread, a long list spreads over many workgroups and a short one stays
// whole.  A row no longer than chunk
// is one item that writes its output directly; a longer row's items write
// consecutive partial rows, listed in `splits` for the combine.  Bounds:
// items <= rows + PLAN_TARGET, split rows < PLAN_TARGET, partial rows
// < 2 * PLAN_TARGET.  A row longer than max_len is one empty item, which the
// forward kernel marks cut (NaN).  This takes the place of the reference's
// get_mla_metadata_kernel (opus_attn/dsa_v32/common/get_mla_metadata.hpp:
// 8-158), which packs per-CU payloads serially; here equal-sized items are
// left to the hardware dispatcher.
// hdr[0] = items, hdr[1] = split rows, hdr[2] = chunk, hdr[3..5] = the B,
// s_q and max_len the plan was built for (checked by the kernels that read
// it).  Item counts per row are computed without int32 overflow for lists up
// to DSA_MLA_MAX_LIST entries.
// ---------------------------------------------------------------------------
constexpr int PLAN_TARGET = 256;     // workgroups a plan aims at: one per CU
constexpr int PLAN_MIN_CHUNK = 128;  // entries: at least four tiles per item
constexpr int PLAN_THREADS = 256;

__global__ void __launch_bounds__(PLAN_THREADS)
dsa_csr_plan_kernel(const int32_t* __restrict__ indptr, int B, int s_q, int max_len, int4* __restrict__ items,
                    int4* __restrict__ splits, int32_t* __restrict__ hdr) {
    constexpr int NW = PLAN_THREADS / 64;
    __shared__ long long s_tot[NW];
    __shared__ int s_scan[3][NW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rows = B * s_q;
    // entries of row q; -1 for a row longer than max_len
    auto len_of = [&](int q) -> int {
        const int b = q / s_q, t = q - b * s_q;
        const int64_t L = (int64_t)indptr[b + 1] - indptr[b] - (s_q - 1 - t);
        return L > max_len ? -1 : (int)max(L, (int64_t)0);
    };
    static_assert(PLAN_TARGET <= PLAN_THREADS, "below PLAN_TARGET rows, one row per thread");
    const bool few = rows < PLAN_TARGET;
    const int Lr = few && tid < rows ? len_of(tid) : 0;    // this thread's row when few
    int chunk;
    if (!few) {
        long long tot = 0;
        for (int q = tid; q < rows; q += PLAN_THREADS) tot += max(len_of(q), 0);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) tot += __shfl_xor(tot, off, 64);
        if (lane == 0) s_tot[wave] = tot;
        __syncthreads();
        long long total = 0;
        for (int w = 0; w < NW; ++w) total += s_tot[w];
        long long c64 = max((long long)PLAN_MIN_CHUNK, (total + PLAN_TARGET - 1) / PLAN_TARGET);
        c64 = (c64 + TILE - 1) / TILE * TILE;
        chunk = (int)min(c64, (long long)MAX_LIST);
    } else {
        // Fewer rows than PLAN_TARGET (one per thread): the smallest chunk, in
        // tiles and >= PLAN_MIN_CHUNK, whose items fit one round of
        // PLAN_TARGET workgroups, sum over rows of ceil(L / chunk) <=
        // PLAN_TARGET (a cut row is one item).  The count falls as chunk
        // grows, and chunk = the longest list gives rows items: bisection.
        __shared__ int s_cnt[NW];
        int lmax = Lr;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) lmax = max(lmax, __shfl_xor(lmax, off, 64));
        if (lane == 0) s_cnt[wave] = lmax;
        __syncthreads();
        for (int w = 0; w < NW; ++w) lmax = max(lmax, s_cnt[w]);
        __syncthreads();
        int lo = PLAN_MIN_CHUNK / TILE, hi = max(lo, (lmax + TILE - 1) / TILE);   // in tiles
        while (lo < hi) {
            const int mid = (lo + hi) / 2, c = mid * TILE;
            int n = tid < rows ? (Lr <= c ? 1 : Lr / c + (Lr % c != 0)) : 0;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) n += __shfl_xor(n, off, 64);
            if (lane == 0) s_cnt[wave] = n;
            __syncthreads();
            int cnt = 0;
            for (int w = 0; w < NW; ++w) cnt += s_cnt[w];
            __syncthreads();
            if (cnt <= PLAN_TARGET) hi = mid;
            else lo = mid + 1;
        }
        chunk = lo * TILE;
    }
    auto wave_incl = [&](int v) {
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int u = __shfl_up(v, off, 64);
            if (lane >= off) v += u;
        }
        return v;
    };
    int item_base = 0, slot_base = 0, split_base = 0;
    for (int q0 = 0; q0 < rows; q0 += PLAN_THREADS) {
        const int q = q0 + tid;
        int L = 0, n = 0;
        if (q < rows) {
            L = few ? Lr : len_of(q);
            n = L <= chunk ? 1 : L / chunk + (L % chunk != 0);
        }
        const int ns = n > 1 ? n : 0, sp = n > 1 ? 1 : 0;
        const int ia = wave_incl(n), ic = wave_incl(ns), id = wave_incl(sp);
        if (lane == 63) {
            s_scan[0][wave] = ia;
            s_scan[1][wave] = ic;
            s_scan[2][wave] = id;
        }
        __syncthreads();
        int wa = 0, wc = 0, wd = 0, ta = 0, tc = 0, td = 0;
        for (int w = 0; w < NW; ++w) {
            const int x = s_scan[0][w], y = s_scan[1][w], z = s_scan[2][w];
            if (w < wave) { wa += x; wc += y; wd += z; }
            ta += x; tc += y; td += z;
        }
        const int ib = item_base + wa + ia - n;
        const int sb = slot_base + wc + ic - ns;
        const int pb = split_base + wd + id - sp;
        for (int j = 0; j < n; ++j) {
            const int e0 = L < 0 ? 0 : j * chunk;
            const int e1 = L < 0 ? 0 : (int)min((int64_t)(j + 1) * chunk, (int64_t)L);
            items[ib + j] = make_int4(q, e0, e1, plan_item_w(n > 1 ? sb + j : -1, j == n - 1));
        }
        if (n > 1) splits[pb] = make_int4(q, sb, n, 0);
        item_base += ta;
        slot_base += tc;
        split_base += td;
        __syncthreads();    // s_scan is rewritten by the next round
    }
    if (tid == 0) {
        hdr[0] = item_base;
        hdr[1] = split_base;
        hdr[2] = chunk;
        hdr[PLAN_HDR_B] = B;
        hdr[PLAN_HDR_SQ] = s_q;
        hdr[PLAN_HDR_MAXLEN] = max_len;
    }
}

// One (query row, head) of a combine, on one wave: ns partial rows, split s
// at partial row first + s * step_rows.  sink (V4 prefill, per head, natural
// log units, or NULL): an attention sink joins the denominator once, here,
// as in the reference's split fold (the splits themselves run without it):
// m = max(lse_i, sink), den = sum w_i + exp(sink - m), so a sink far above
// or below every score neither overflows nor underflows.  A row with no
// attended entry keeps O = 0 and LSE = +inf, as unsplit.
// splits a wave merges with all its loads in flight at once
constexpr int SMALL_SPLITS = 16;
__device__ __forceinline__ void combine_head(const float* __restrict__ part_o, const float* __restrict__ part_lse,
                                             int ns, int64_t first, int64_t step_rows, int row, int head, int H,
                                             int s_q, __bf16* __restrict__ out, int64_t o_sb, int64_t o_st,
                                             int64_t o_sh, float* __restrict__ lse, const float* __restrict__ sink,
                                             int lane) {
    const int64_t stride = step_rows * H;
    const int64_t base = first * H + head;     // partial index of split 0
    const int64_t rh = (int64_t)row * H + head;
    float m = -FLT_MAX;
    f32x4 acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    float den = 0.0f;
    bool sink_on;
    float sk;
    if (ns <= SMALL_SPLITS) {
        // Every split's LSE and O slice loaded at once: one memory round trip
        // (the general path below needs one for the maximum, then one per
        // eight splits).  The same maximum and the same sums in split order.
        float ls[SMALL_SPLITS];
        f32x4 v[SMALL_SPLITS][2];
#pragma unroll
        for (int j = 0; j < SMALL_SPLITS; ++j) {
            if (j < ns) {
                ls[j] = part_lse[j * stride + base];
                const f32x4* src = reinterpret_cast<const f32x4*>(part_o + (j * stride + base) * D_VO + 8 * lane);
                v[j][0] = src[0];
                v[j][1] = src[1];
            }
        }
#pragma unroll
        for (int j = 0; j < SMALL_SPLITS; ++j)
            if (j < ns) m = fmaxf(m, ls[j]);
        sink_on = sink != nullptr && m > -FLT_MAX;
        sk = sink_on ? sink[head] : 0.0f;
        if (sink_on) m = fmaxf(m, sk);
#pragma unroll
        for (int j = 0; j < SMALL_SPLITS; ++j) {
            if (j < ns) {
                const float w = ls[j] > -FLT_MAX || ls[j] != ls[j] ? __builtin_amdgcn_exp2f((ls[j] - m) * LOG2E) : 0.0f;
                den += w;
                acc0 += w * v[j][0];
                acc1 += w * v[j][1];
            }
        }
        ns = 0;       // (the loop below has nothing left to do)
    } else {
        for (int s = lane; s < ns; s += 64) m = fmaxf(m, part_lse[s * stride + base]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        sink_on = sink != nullptr && m > -FLT_MAX;
        sk = sink_on ? sink[head] : 0.0f;
        if (sink_on) m = fmaxf(m, sk);
    }
    // eight splits' loads in flight at a time; sums in split order
    for (int s0 = 0; s0 < ns; s0 += 8) {
        float ls[8];
        f32x4 v[8][2];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (s0 + j < ns) {
                ls[j] = part_lse[(s0 + j) * stride + base];
                const f32x4* src = reinterpret_cast<const f32x4*>(part_o + ((s0 + j) * stride + base) * D_VO + 8 * lane);
                v[j][0] = src[0];
                v[j][1] = src[1];
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (s0 + j < ns) {
                // an empty split (-FLT_MAX) weighs 0; a NaN LSE (a list cut
                // short) makes the row NaN
                const float w = ls[j] > -FLT_MAX || ls[j] != ls[j] ? __builtin_amdgcn_exp2f((ls[j] - m) * LOG2E) : 0.0f;
                den += w;
                acc0 += w * v[j][0];
                acc1 += w * v[j][1];
            }
        }
    }
    if (sink_on) den += __builtin_amdgcn_exp2f((sk - m) * LOG2E);
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    const bf16x4 b0 = __builtin_convertvector(acc0 * inv, bf16x4);
    const bf16x4 b1 = __builtin_convertvector(acc1 * inv, bf16x4);
    __bf16* op = out + (int64_t)(row / s_q) * o_sb + (int64_t)(row % s_q) * o_st + (int64_t)head * o_sh + 8 * lane;
    reinterpret_cast<u32x2*>(op)[0] = __builtin_bit_cast(u32x2, b0);
    reinterpret_cast<u32x2*>(op)[1] = __builtin_bit_cast(u32x2, b1);
    if (lse && lane == 0) lse[rh] = den > 0.0f || den != den ? m + __builtin_amdgcn_logf(den) * LN2 : INFINITY;
}

constexpr int COMBINE_MAX_Y = 65535;     // the grid's y extent (HIP's limit is 65536)

// uniform splits: split s of row r is partial row s * rows + r.
// grid = (rows, min(H, COMBINE_MAX_Y)), block = 64: one workgroup of one wave
// per (row, head), so that a low-batch call's few rows still spread over every
// CU (four heads per workgroup put C1's 256 (row, head) pairs on 64 CUs, each
// pulling 128 KB of partials through its own memory path).  Past
// COMBINE_MAX_Y heads a workgroup takes every gridDim.y-th head.
__global__ void __launch_bounds__(64)
dsa_mla_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_lse, int ns,
                       int rows, int H, int s_q, __bf16* __restrict__ out, int64_t o_sb, int64_t o_st,
                       int64_t o_sh, float* __restrict__ lse, const float* __restrict__ sink) {
    const int row = blockIdx.x;
    for (int head = blockIdx.y; head < H; head += gridDim.y)
        combine_head(part_o, part_lse, ns, row, rows, row, head, H, s_q, out, o_sb, o_st, o_sh, lse, sink,
                     threadIdx.x & 63);
}

// The split rows of a CSR work plan: map[i] = (query row, first partial row,
// count), consecutive partial rows, hdr[1] rows listed.  A fixed grid walks
// the hdr[1] x ceil(H / 4) units of four heads, so a plan without split rows
// costs one wave of empty workgroups, not a workgroup per possible unit.
__global__ void __launch_bounds__(256)
dsa_mla_combine_plan_kernel(const float* __restrict__ part_o, const float* __restrict__ part_lse, int B, int H,
                            int s_q, int max_len, __bf16* __restrict__ out, int64_t o_sb, int64_t o_st,
                            int64_t o_sh, float* __restrict__ lse, const int4* __restrict__ map,
                            const int32_t* __restrict__ hdr) {
    // a plan built for other arguments: the forward kernel has written NaN rows
    if (__builtin_amdgcn_readfirstlane(hdr[PLAN_HDR_B]) != B ||
        __builtin_amdgcn_readfirstlane(hdr[PLAN_HDR_SQ]) != s_q ||
        __builtin_amdgcn_readfirstlane(hdr[PLAN_HDR_MAXLEN]) != max_len)
        return;
    const int hq = (H + 3) / 4;
    const int units = __builtin_amdgcn_readfirstlane(hdr[1]) * hq;
    const int wave = threadIdx.x >> 6;
    for (int u = blockIdx.x; u < units; u += gridDim.x) {
        const int r = u / hq;
        const int head = (u - r * hq) * 4 + wave;
        if (head < H) {
            const int4 m = map[r];
            combine_head(part_o, part_lse, m.z, m.y, 1, m.x, head, H, s_q, out, o_sb, o_st, o_sh, lse, nullptr,
                         threadIdx.x & 63);
        }
    }
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

int decode_launch(const dsa_mla_decode_args* a, int ns, int chunk, void* ws, hipStream_t st);

// Device scratch of dsa_mla_decode_noalloc: the split partials (fp32 O and
// LSE) of a call live here instead of in a caller workspace.  Every GPU the
// library runs on holds its own copy for the life of the process.  The name is
// only a host-side handle: host code uses the per-device address that
// hipGetSymbolAddress returns, never the array's name.  Nothing in it must
// start at zero (every split writes all its partials before the combine reads
// them); calls that overlap on one GPU share it and race.
static __device__ __align__(256) unsigned char scratch[DSA_MLA_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
void* g_scratch_ptr[MAX_DEVICES];
std::mutex g_scratch_mu;

// The current device's address of `scratch`, looked up once per device (with
// that device current, which it is: it is the current device).
int device_scratch(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return DSA_ERR_HIP;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return DSA_ERR_HIP;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DSA_OK;
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Bytes between cache rows for a row stride given in elements of the row
// format's storage type (bf16 elements, or bytes for 656-B rows); 0 = dense.
// -1 when the stride is shorter than a row or not a multiple of 16 bytes
// (every gather load is 16 bytes).
int64_t row_stride_bytes(int fmt, int64_t stride) {
    const int64_t dense = fmt == DSA_KV_FP8_656 ? FP8_ROW : BF16_ROW;
    if (stride == 0) return dense;
    const int64_t bytes = fmt == DSA_KV_FP8_656 ? stride : 2 * stride;
    // (below 4 GiB: the kernels form a row's byte offset as a 32 x 32-bit product)
    return stride < 0 || bytes < dense || (bytes % 16) != 0 || bytes > 0xFFFFFFF0ll ? -1 : bytes;
}
int ilog2(int v) { int s = 0; while ((1 << s) < v) ++s; return s; }
// workgroups per query token: 128 heads each (the last group masks heads past H)
int head_groups(int32_t H) { return (H + HEADS - 1) / HEADS; }
// any H >= 1; the grid's x extent (query tokens x head groups) stays below 2^31
bool heads_ok(int32_t H, int64_t tokens) {
    return H >= 1 && tokens * head_groups(H) <= INT32_MAX;
}

// Forward kernel for bf16 rows (576-value rows in the top-k or uniform-split
// CSR form, V4 512-value rows) and 656-B fp8 rows (the same forms):
// 32-head workgroups (dsa_mla_fwd_narrow_kernel) when the 128-head kernel
// would compute at least 4x padding heads (H <= 32), or could not occupy half
// the GPU even with its splits (fewer than 128 workgroups at wide_splits
// splits).  Per head and row the 32-head kernel costs about 2.3x the cycles,
// so it pays only where the 128-head kernel leaves CUs idle or computes
// mostly padding.
int narrow_groups(int32_t H) { return (H + NARROW_HEADS - 1) / NARROW_HEADS; }
bool narrow_path(int fmt, int64_t tokens, int32_t H, int wide_splits) {
    if ((fmt != DSA_KV_BF16 && fmt != DSA_KV_BF16_D512 && fmt != DSA_KV_FP8_656) || H < 1 ||
        tokens * narrow_groups(H) > INT32_MAX)
        return false;
    return H <= 32 || tokens * head_groups(H) * wide_splits < 128;
}

int auto_splits(int64_t queries, int topk) {
    int ns = 1;
    if (queries > 0 && queries < 256) {
        const int64_t want = (256 + queries - 1) / queries;
        // keep >= 4 tiles per split (at top-k 2048 and B = 2 or 4: 16 splits
        // measured 11 % faster than 8 and 6 % faster than 32)
        const int64_t by_len = (topk + 127) / 128;
        ns = (int)std::min<int64_t>(want, std::max<int64_t>(1, by_len));
    }
    return std::min(ns, DSA_MLA_MAX_SPLITS);
}

// Split count and kernel of a top-k decode call: the caller's count, or the
// automatic one for the kernel narrow_path picks.
int decode_splits(const dsa_mla_decode_args* a, bool* narrow) {
    const int64_t tokens = (int64_t)a->B * a->s_q;
    const int wide = a->num_splits ? a->num_splits : auto_splits(tokens * head_groups(a->H), a->topk);
    *narrow = narrow_path(a->kv_format, tokens, a->H, wide);
    if (a->num_splits || !*narrow) return wide;
    return auto_splits(tokens * narrow_groups(a->H), a->topk);
}

int validate_decode(const dsa_mla_decode_args* a, int* ns_out, int* chunk_out) {
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->B < 0 || a->s_q <= 0 || a->topk < 0 || a->topk > MAX_LIST) return DSA_ERR_BAD_SHAPE;
    if (!heads_ok(a->H, a->B)) return DSA_ERR_BAD_SHAPE;
    if (a->kv_format != DSA_KV_BF16 && a->kv_format != DSA_KV_FP8_656) return DSA_ERR_BAD_FORMAT;
    if (a->kv_total_rows < 0 || a->kv_total_rows > INT32_MAX) return DSA_ERR_BAD_SHAPE;
    if (a->block_table && a->block_size <= 0) return DSA_ERR_BAD_SHAPE;
    if (row_stride_bytes(a->kv_format, a->kv_stride_row) < 0) return DSA_ERR_BAD_STRIDE;
    if (a->num_splits < 0 || a->num_splits > DSA_MLA_MAX_SPLITS) return DSA_ERR_BAD_SPLITS;
    bool narrow;
    const int ns = decode_splits(a, &narrow);
    const int chunk = a->topk == 0 ? 0 : (a->topk + ns - 1) / ns;
    if (a->B > 0 && a->topk > 0) {
        if (!a->q || !a->kv_cache || !a->seq_lens || !a->indices || !a->out) return DSA_ERR_NULL_POINTER;
        if ((a->q_stride_h % 8) != 0 || (a->q_stride_t % 8) != 0 || (a->q_stride_b % 8) != 0)
            return DSA_ERR_BAD_STRIDE;
        if ((a->o_stride_h % 4) != 0 || (a->o_stride_t % 4) != 0 || (a->o_stride_b % 4) != 0)
            return DSA_ERR_BAD_STRIDE;
        if (((uintptr_t)a->q & 15) || ((uintptr_t)a->kv_cache & 15) || ((uintptr_t)a->out & 7))
            return DSA_ERR_BAD_STRIDE;
    }
    // the kernel reads Q even when no entry is valid: q is needed whenever B > 0
    if (a->B > 0 && a->topk == 0 && (!a->out || !a->q)) return DSA_ERR_NULL_POINTER;
    *ns_out = ns;
    *chunk_out = chunk;
    return DSA_OK;
}

size_t decode_ws_bytes(const dsa_mla_decode_args* a, int ns) {
    if (ns <= 1 || a->B == 0) return 0;
    const size_t rows = (size_t)a->B * a->s_q * a->H;
    return (size_t)ns * rows * (D_VO + 1) * sizeof(float) + 256;
}

int launch_fwd(const FwdParams& fp, int fmt, int B, int s_q, int ns, hipStream_t st, bool narrow = false) {
    dim3 grid((unsigned)((int64_t)B * fp.hgroups), s_q, ns), block(NTHR);
    if (narrow && fmt == DSA_KV_BF16_D512)
        hipLaunchKernelGGL(dsa_mla_fwd_narrow_kernel<DSA_KV_BF16_D512>, grid, block, 0, st, fp);
    else if (narrow && fmt == DSA_KV_FP8_656)
        hipLaunchKernelGGL(dsa_mla_fwd_narrow_kernel<DSA_KV_FP8_656>, grid, block, 0, st, fp);
    else if (narrow) hipLaunchKernelGGL(dsa_mla_fwd_narrow_kernel<DSA_KV_BF16>, grid, block, 0, st, fp);
    else if (fmt == DSA_KV_BF16) hipLaunchKernelGGL(dsa_mla_fwd_kernel<DSA_KV_BF16>, grid, block, 0, st, fp);
    else if (fmt == DSA_KV_FP8_656) hipLaunchKernelGGL(dsa_mla_fwd_kernel<DSA_KV_FP8_656>, grid, block, 0, st, fp);
    else if (fmt == DSA_KV_MXFP8) hipLaunchKernelGGL(dsa_mla_fwd_kernel<DSA_KV_MXFP8>, grid, block, 0, st, fp);
    else if (fmt == DSA_KV_MXFP8_V4) hipLaunchKernelGGL(dsa_mla_fwd_kernel<DSA_KV_MXFP8_V4>, grid, block, 0, st, fp);
    else hipLaunchKernelGGL(dsa_mla_fwd_kernel<DSA_KV_BF16_D512>, grid, block, 0, st, fp);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

int launch_combine(const float* po, const float* pl, int ns, int rows, int H, int s_q, void* out, int64_t o_sb,
                   int64_t o_st, int64_t o_sh, float* lse, hipStream_t st, const float* sink = nullptr) {
    if (rows == 0) return DSA_OK;
    dim3 grid(rows, std::min(H, COMBINE_MAX_Y)), block(64);
    hipLaunchKernelGGL(dsa_mla_combine_kernel, grid, block, 0, st, po, pl, ns, rows, H, s_q, (__bf16*)out, o_sb,
                       o_st, o_sh, lse, sink);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

// Workspace of a CSR work plan: header, item table, split-row map, then the
// partial rows (fp32 O, then LSE).  A row is split only when it is longer than
// the plan's chunk (>= PLAN_MIN_CHUNK entries), and a plan never holds more than
// 2 * PLAN_TARGET partial rows.
struct CsrPlanLayout {
    size_t items, map, po, pl, total;
    int items_max, slots_max;
};
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
CsrPlanLayout csr_plan_layout(int B, int s_q, int H, int max_len) {
    CsrPlanLayout L{};
    const int64_t rows = (int64_t)B * s_q;
    L.items_max = (int)(rows + PLAN_TARGET);
    const int64_t per_row = ((int64_t)max_len + PLAN_MIN_CHUNK - 1) / PLAN_MIN_CHUNK;
    L.slots_max = max_len > PLAN_MIN_CHUNK ? (int)std::min<int64_t>(2 * PLAN_TARGET, rows * per_row) : 0;
    L.items = 256;
    L.map = align256(L.items + (size_t)L.items_max * sizeof(int4));
    L.po = align256(L.map + (size_t)PLAN_TARGET * sizeof(int4));
    L.pl = align256(L.po + (size_t)L.slots_max * H * D_VO * sizeof(float));
    L.total = align256(L.pl + (size_t)L.slots_max * H * sizeof(float));
    return L;
}
// the plan's grid: (rows + PLAN_TARGET) x head groups workgroups
bool plan_grid_ok(int B, int s_q, int H) {
    return ((int64_t)B * s_q + PLAN_TARGET) * head_groups(H) <= INT32_MAX - PLAN_THREADS;
}
// the plan kernel alone (into a workspace laid out by csr_plan_layout)
int csr_plan_build(const int32_t* kv_indptr, int B, int s_q, int H, int max_len, void* ws, hipStream_t st) {
    const CsrPlanLayout L = csr_plan_layout(B, s_q, H, max_len);
    char* w = (char*)ws;
    hipLaunchKernelGGL(dsa_csr_plan_kernel, dim3(1), dim3(PLAN_THREADS), 0, st, kv_indptr, B, s_q, max_len,
                       (int4*)(w + L.items), (int4*)(w + L.map), (int32_t*)w);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}
// (plan kernel,) forward kernel over the plan's items, combine of the split rows;
// build = false: the workspace already holds the plan of these lists
int csr_plan_launch(FwdParams& fp, int fmt, int max_len, void* ws, bool build, hipStream_t st) {
    const CsrPlanLayout L = csr_plan_layout(fp.B, fp.s_q, fp.H, max_len);
    char* w = (char*)ws;
    int32_t* hdr = (int32_t*)w;
    int4* items = (int4*)(w + L.items);
    int4* map = (int4*)(w + L.map);
    if (build) {
        const int r = csr_plan_build(fp.kv_indptr, fp.B, fp.s_q, fp.H, max_len, ws, st);
        if (r) return r;
    }
    fp.plan_items = items;
    fp.plan_hdr = hdr;
    fp.chunk = max_len;      // one launch "split": lists longer than max_len are cut
    if (L.slots_max) {
        fp.part_o = (float*)(w + L.po);
        fp.part_lse = (float*)(w + L.pl);
    }
    // (a multiple of 8 s_q workgroups: the item order the kernel maps them to)
    const int G = 8 * fp.s_q;
    const int r = launch_fwd(fp, fmt, (L.items_max + G - 1) / G * G, 1, 1, st);
    if (r || !L.slots_max) return r;
    hipLaunchKernelGGL(dsa_mla_combine_plan_kernel, dim3(4 * PLAN_TARGET), dim3(256), 0, st, (const float*)fp.part_o,
                       (const float*)fp.part_lse, fp.B, fp.H, fp.s_q, max_len, fp.out, fp.o_sb, fp.o_st, fp.o_sh,
                       fp.lse, (const int4*)map, (const int32_t*)hdr);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

int validate_csr(const dsa_mla_decode_csr_args* a, int* ns_out, int* chunk_out) {
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->B < 0 || a->s_q <= 0 || a->max_kv_len < 0 || a->max_kv_len > MAX_LIST || a->total_tokens < 0)
        return DSA_ERR_BAD_SHAPE;
    if (!heads_ok(a->H, a->B)) return DSA_ERR_BAD_SHAPE;
    if (a->kv_format != DSA_KV_BF16 && a->kv_format != DSA_KV_FP8_656) return DSA_ERR_BAD_FORMAT;
    if (row_stride_bytes(a->kv_format, a->stride_kv_page) < 0) return DSA_ERR_BAD_STRIDE;
    if (a->num_splits < DSA_MLA_SPLITS_PLANNED || a->num_splits > DSA_MLA_MAX_SPLITS) return DSA_ERR_BAD_SPLITS;
    // num_splits 0: build the device work plan; DSA_MLA_SPLITS_PLANNED: the
    // workspace holds it (dsa_mla_csr_plan); else uniform splits
    const int ns = a->num_splits;
    if (ns <= 0 && !plan_grid_ok(a->B, a->s_q, a->H)) return DSA_ERR_BAD_SHAPE;
    const int chunk = a->max_kv_len == 0 || ns <= 0 ? a->max_kv_len : (a->max_kv_len + ns - 1) / ns;
    if (a->B > 0) {
        // the kernel reads Q even when every list is empty
        if (!a->out || !a->kv_indptr || !a->q) return DSA_ERR_NULL_POINTER;
        if (a->max_kv_len > 0 && (!a->kv || !a->kv_indices)) return DSA_ERR_NULL_POINTER;
        if (a->stride_q_b < 0 || a->stride_q_h < 0 || a->stride_o_b < 0 || a->stride_o_h < 0)
            return DSA_ERR_BAD_STRIDE;
        if ((a->stride_q_h % 8) || (a->stride_q_b % 8) || (a->stride_o_h % 4) || (a->stride_o_b % 4))
            return DSA_ERR_BAD_STRIDE;
        if (((uintptr_t)a->q & 15) || ((uintptr_t)a->kv & 15) || ((uintptr_t)a->out & 7))
            return DSA_ERR_BAD_STRIDE;
    }
    *ns_out = ns;
    *chunk_out = chunk;
    return DSA_OK;
}
size_t csr_ws_bytes(const dsa_mla_decode_csr_args* a, int ns) {
    if (a->B == 0) return 0;
    if (ns <= 0) return csr_plan_layout(a->B, a->s_q, a->H, a->max_kv_len).total;
    return ns == 1 ? 0 : (size_t)ns * a->B * a->s_q * a->H * (D_VO + 1) * sizeof(float) + 256;
}

int validate_mx(const dsa_mla_decode_mxfp8_args* a, int* ns_out, int* chunk_out) {
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->B < 0 || a->s_q <= 0 || a->max_kv_len < 0 || a->max_kv_len > MAX_LIST || a->total_tokens < 0)
        return DSA_ERR_BAD_SHAPE;
    if (!heads_ok(a->H, a->B)) return DSA_ERR_BAD_SHAPE;
    if (a->num_splits < DSA_MLA_SPLITS_PLANNED || a->num_splits > DSA_MLA_MAX_SPLITS) return DSA_ERR_BAD_SPLITS;
    // num_splits 0: build the device work plan; DSA_MLA_SPLITS_PLANNED: the
    // workspace holds it (dsa_mla_csr_plan); else uniform splits
    const int ns = a->num_splits;
    if (ns <= 0 && !plan_grid_ok(a->B, a->s_q, a->H)) return DSA_ERR_BAD_SHAPE;
    const int chunk = a->max_kv_len == 0 || ns <= 0 ? a->max_kv_len : (a->max_kv_len + ns - 1) / ns;
    if (a->B > 0) {
        // the kernel reads Q even when every list is empty
        if (!a->out || !a->kv_indptr || !a->q_nope || !a->q_scale || !a->q_rope) return DSA_ERR_NULL_POINTER;
        if (a->max_kv_len > 0 && (!a->kv_nope || !a->kv_scale || !a->kv_rope || !a->kv_indices))
            return DSA_ERR_NULL_POINTER;
        // fp8 / E8M0 streams: bytes, multiples of 16; bf16 streams: multiples of 8 elements
        const int32_t b16[] = {a->stride_q_nope_b, a->stride_q_nope_h, a->stride_q_scale_b, a->stride_q_scale_h,
                               a->stride_kv_nope_page, a->stride_kv_scale_page};
        const int32_t e8[] = {a->stride_q_rope_b, a->stride_q_rope_h, a->stride_kv_rope_page};
        for (int32_t v : b16) if (v < 0 || (v % 16)) return DSA_ERR_BAD_STRIDE;
        for (int32_t v : e8) if (v < 0 || (v % 8)) return DSA_ERR_BAD_STRIDE;
        if (a->stride_o_b < 0 || a->stride_o_h < 0 || (a->stride_o_b % 4) || (a->stride_o_h % 4))
            return DSA_ERR_BAD_STRIDE;
        const void* ptrs[] = {a->q_nope, a->q_scale, a->q_rope, a->kv_nope, a->kv_scale, a->kv_rope};
        for (const void* q : ptrs) if ((uintptr_t)q & 15) return DSA_ERR_BAD_STRIDE;
        if ((uintptr_t)a->out & 7) return DSA_ERR_BAD_STRIDE;
    }
    *ns_out = ns;
    *chunk_out = chunk;
    return DSA_OK;
}
size_t mx_ws_bytes(const dsa_mla_decode_mxfp8_args* a, int ns) {
    if (a->B == 0) return 0;
    if (ns <= 0) return csr_plan_layout(a->B, a->s_q, a->H, a->max_kv_len).total;
    return ns == 1 ? 0 : (size_t)ns * a->B * a->s_q * a->H * (D_VO + 1) * sizeof(float) + 256;
}

// Splits of a prefill: num_splits when given, else (0) more than one only when
// fewer than 256 workgroups (query tokens x head groups) would run, keeping at
// least 8 tiles (256 entries of the longest list) per split.  A token's
// split s covers its list's part s of whole tiles; the partials are merged by
// the combine kernel (with the attention sink, V4).
// Split count and kernel of a prefill call (N query tokens, lists of at most
// max_list entries).
int prefill_plan(int fmt, int64_t N, int32_t H, int requested, int64_t max_list, bool* narrow);
int prefill_splits(int requested, int64_t wgs, int64_t max_list) {
    if (requested > 0) return requested;
    if (wgs <= 0 || wgs >= 256) return 1;
    const int64_t want = (256 + wgs - 1) / wgs;
    const int64_t by_len = std::max<int64_t>(1, max_list / 256);
    return (int)std::min<int64_t>(std::min<int64_t>(want, by_len), DSA_MLA_MAX_SPLITS);
}
int prefill_plan(int fmt, int64_t N, int32_t H, int requested, int64_t max_list, bool* narrow) {
    const int wide = prefill_splits(requested, N * head_groups(H), max_list);
    *narrow = narrow_path(fmt, N, H, wide);
    return *narrow ? prefill_splits(requested, N * narrow_groups(H), max_list) : wide;
}
size_t prefill_ws_bytes(int ns, int64_t N, int H) {
    return ns <= 1 || N == 0 ? 0 : (size_t)ns * N * H * (D_VO + 1) * sizeof(float) + 256;
}
// Forward kernel over ns splits of N query tokens, then (ns > 1) the combine of
// their partials, with the attention sink folded in once by the combine.
int prefill_launch(FwdParams& fp, int fmt, int ns, const float* sink, void* ws, hipStream_t st,
                   bool narrow = false) {
    const int64_t N = fp.B;
    if (ns > 1) {
        fp.part_o = (float*)ws;
        fp.part_lse = (float*)((char*)ws + (size_t)ns * N * fp.H * D_VO * sizeof(float));
        fp.attn_sink = nullptr;
    } else {
        fp.attn_sink = sink;
    }
    const int r = launch_fwd(fp, fmt, (int)N, 1, ns, st, narrow);
    if (r || ns == 1) return r;
    return launch_combine(fp.part_o, fp.part_lse, ns, (int)N, fp.H, 1, fp.out, fp.o_sb, 0, fp.o_sh, fp.lse, st,
                          sink);
}

int validate_prefill(const dsa_mla_prefill_args* a, int* ns_out) {
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->N < 0 || a->topk < 0 || a->kv_rows < 0 || a->kv_rows > INT32_MAX) return DSA_ERR_BAD_SHAPE;
    if (!heads_ok(a->H, a->N)) return DSA_ERR_BAD_SHAPE;
    if (a->kv_format != DSA_KV_BF16 && a->kv_format != DSA_KV_FP8_656) return DSA_ERR_BAD_FORMAT;
    if (row_stride_bytes(a->kv_format, a->kv_stride_row) < 0) return DSA_ERR_BAD_STRIDE;
    if (a->topk > MAX_LIST) return DSA_ERR_BAD_SHAPE;
    if (a->num_splits < 0 || a->num_splits > DSA_MLA_MAX_SPLITS) return DSA_ERR_BAD_SPLITS;
    bool narrow;
    *ns_out = prefill_plan(a->kv_format, a->N, a->H, a->num_splits, a->topk, &narrow);
    if (a->N == 0) return DSA_OK;
    if (!a->q || !a->out || (a->topk > 0 && (!a->kv || !a->indices))) return DSA_ERR_NULL_POINTER;
    if ((a->q_stride_n % 8) || (a->q_stride_h % 8) || (a->o_stride_n % 4) || (a->o_stride_h % 4))
        return DSA_ERR_BAD_STRIDE;
    if (((uintptr_t)a->q & 15) || ((uintptr_t)a->kv & 15) || ((uintptr_t)a->out & 7)) return DSA_ERR_BAD_STRIDE;
    return DSA_OK;
}

int validate_v4(const dsa_mla_prefill_v4_args* a, int* ns_out) {
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->N < 0 || a->total_pages < 0 || a->total_tokens < 0 || a->max_rows < 0) return DSA_ERR_BAD_SHAPE;
    // row ids carry their pool in bit 30 (dsa_rows.h): each pool stays below 2^30 rows
    if (a->total_pages >= dsa_rows::MAX_POOL_ROWS || a->total_tokens >= dsa_rows::MAX_POOL_ROWS)
        return DSA_ERR_BAD_SHAPE;
    if (a->max_rows > MAX_LIST) return DSA_ERR_BAD_SHAPE;
    if (!heads_ok(a->H, a->N)) return DSA_ERR_BAD_SHAPE;
    if (a->D != DSA_MLA_D_V4) return DSA_ERR_UNSUPPORTED;
    if (a->num_splits < 0 || a->num_splits > DSA_MLA_MAX_SPLITS) return DSA_ERR_BAD_SPLITS;
    bool narrow;
    *ns_out = prefill_plan(DSA_KV_BF16_D512, a->N, a->H, a->num_splits, a->max_rows, &narrow);
    if (a->N == 0) return DSA_OK;
    if (!a->q || !a->out || !a->kv_indptr_prefix || !a->kv_indices_prefix || !a->kv_indptr_extend ||
        !a->kv_indices_extend)
        return DSA_ERR_NULL_POINTER;
    if ((a->total_pages > 0 && !a->unified_kv) || (a->total_tokens > 0 && !a->kv)) return DSA_ERR_NULL_POINTER;
    if (a->stride_qo_n < 0 || a->stride_qo_h < 0 || (a->stride_qo_n % 8) || (a->stride_qo_h % 8) ||
        a->stride_kv_page < DSA_MLA_D_V4 || (a->stride_kv_page % 8))
        return DSA_ERR_BAD_STRIDE;
    if (((uintptr_t)a->q & 15) || ((uintptr_t)a->unified_kv & 15) || ((uintptr_t)a->kv & 15) ||
        ((uintptr_t)a->out & 7))
        return DSA_ERR_BAD_STRIDE;
    return DSA_OK;
}

int validate_v4fp8(const dsa_mla_prefill_v4_fp8_args* a, int* ns_out) {
    if (!a) return DSA_ERR_NULL_POINTER;
    if (a->N < 0 || a->total_pages < 0 || a->total_tokens < 0 || a->max_rows < 0) return DSA_ERR_BAD_SHAPE;
    if (a->total_pages >= dsa_rows::MAX_POOL_ROWS || a->total_tokens >= dsa_rows::MAX_POOL_ROWS)
        return DSA_ERR_BAD_SHAPE;
    if (a->max_rows > MAX_LIST) return DSA_ERR_BAD_SHAPE;
    if (!heads_ok(a->H, a->N)) return DSA_ERR_BAD_SHAPE;
    if (a->num_splits < 0 || a->num_splits > DSA_MLA_MAX_SPLITS) return DSA_ERR_BAD_SPLITS;
    *ns_out = prefill_splits(a->num_splits, (int64_t)a->N * head_groups(a->H), a->max_rows);
    if (a->N == 0) return DSA_OK;
    if (!a->q_nope || !a->q_rope || !a->out || !a->kv_indptr_prefix || !a->kv_indices_prefix ||
        !a->kv_indptr_extend || !a->kv_indices_extend)
        return DSA_ERR_NULL_POINTER;
    if ((a->total_pages > 0 && (!a->unified_kv_nope || !a->unified_kv_rope)) ||
        (a->total_tokens > 0 && (!a->kv_nope || !a->kv_rope)))
        return DSA_ERR_NULL_POINTER;
    const int32_t b16[] = {a->stride_q_nope_n, a->stride_q_nope_h, a->stride_kv_nope_page};
    for (int32_t v : b16) if (v < 0 || (v % 16)) return DSA_ERR_BAD_STRIDE;
    if (a->stride_kv_nope_page < DSA_MLA_V4_NOPE_BYTES) return DSA_ERR_BAD_STRIDE;
    const int32_t e8[] = {a->stride_q_rope_n, a->stride_q_rope_h, a->stride_kv_rope_page};
    for (int32_t v : e8) if (v < 0 || (v % 8)) return DSA_ERR_BAD_STRIDE;
    if (a->stride_o_n < 0 || a->stride_o_h < 0 || (a->stride_o_n % 4) || (a->stride_o_h % 4))
        return DSA_ERR_BAD_STRIDE;
    const void* ptrs[] = {a->q_nope, a->q_rope, a->unified_kv_nope, a->unified_kv_rope, a->kv_nope, a->kv_rope};
    for (const void* q : ptrs) if ((uintptr_t)q & 15) return DSA_ERR_BAD_STRIDE;
    if ((uintptr_t)a->out & 7) return DSA_ERR_BAD_STRIDE;
    return DSA_OK;
}

}  // namespace

extern "C" {

int dsa_mla_abi_version(void) { return 8; }

const char* dsa_mla_strerror(int code) {
    switch (code) {
    case DSA_OK: return "success";
    case DSA_ERR_NULL_POINTER: return "a required pointer is NULL";
    case DSA_ERR_BAD_SHAPE: return "invalid shape argument";
    case DSA_ERR_UNSUPPORTED:
        return "unsupported configuration (V4 prefill head dim D other than 512, or an indexer head count "
               "other than 32, 64 or 128)";
    case DSA_ERR_BAD_FORMAT: return "unknown kv_format";
    case DSA_ERR_WORKSPACE: return "workspace missing or too small";
    case DSA_ERR_BAD_SPLITS: return "num_splits out of range or too small for top-k";
    case DSA_ERR_BAD_STRIDE: return "misaligned pointer or stride";
    case DSA_ERR_HIP: return "HIP runtime error";
    case DSA_ERR_SCRATCH_LIMIT:
        return "the call's split partials exceed the no-allocation entry's device scratch "
               "(DSA_MLA_NOALLOC_SCRATCH_BYTES); call dsa_mla_decode with a workspace";
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
    return decode_launch(a, ns, chunk, ws, (hipStream_t)stream);
}

int dsa_mla_decode_noalloc(const dsa_mla_decode_args* a, void* stream) {
    int ns, chunk;
    const int rc = validate_decode(a, &ns, &chunk);
    if (rc) return rc;
    const size_t need = decode_ws_bytes(a, ns);
    if (need > DSA_MLA_NOALLOC_SCRATCH_BYTES) return DSA_ERR_SCRATCH_LIMIT;
    if (a->B == 0) return DSA_OK;
    void* ws = nullptr;
    if (need) {
        const int rs = device_scratch(&ws);
        if (rs) return rs;
    }
    return decode_launch(a, ns, chunk, ws, (hipStream_t)stream);
}

}  // extern "C"

namespace {

int decode_launch(const dsa_mla_decode_args* a, int ns, int chunk, void* ws, hipStream_t st) {
    bool narrow;
    decode_splits(a, &narrow);
    FwdParams fp{};
    fp.H = a->H;
    fp.hgroups = narrow ? narrow_groups(a->H) : head_groups(a->H);
    fp.q = (const __bf16*)a->q;
    fp.q_sb = a->q_stride_b; fp.q_st = a->q_stride_t; fp.q_sh = a->q_stride_h;
    fp.kv = (const unsigned char*)a->kv_cache;
    fp.kv_total_rows = a->kv_total_rows;
    fp.kv_batch_stride = a->kv_batch_stride;
    fp.row_bytes = row_stride_bytes(a->kv_format, a->kv_stride_row);
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
        const size_t rows = (size_t)a->B * a->s_q * a->H;
        fp.part_o = (float*)ws;
        fp.part_lse = (float*)((char*)ws + (size_t)ns * rows * D_VO * sizeof(float));
    }
    int r = launch_fwd(fp, a->kv_format, a->B, a->s_q, ns, st, narrow);
    if (r || ns == 1) return r;
    return launch_combine(fp.part_o, fp.part_lse, ns, a->B * a->s_q, a->H, a->s_q, a->out, a->o_stride_b,
                          a->o_stride_t, a->o_stride_h, a->lse, st);
}

}  // namespace

extern "C" {

int dsa_mla_csr_plan(const int32_t* kv_indptr, int32_t B, int32_t s_q, int32_t H, int32_t max_kv_len, void* ws,
                     size_t ws_bytes, void* stream) {
    if (B < 0 || s_q <= 0 || max_kv_len < 0 || max_kv_len > MAX_LIST) return DSA_ERR_BAD_SHAPE;
    if (!heads_ok(H, B) || !plan_grid_ok(B, s_q, H)) return DSA_ERR_BAD_SHAPE;
    if (B == 0) return DSA_OK;
    if (!kv_indptr) return DSA_ERR_NULL_POINTER;
    const size_t need = csr_plan_layout(B, s_q, H, max_kv_len).total;
    if (!ws || ws_bytes < need || ((uintptr_t)ws & 15)) return DSA_ERR_WORKSPACE;
    return csr_plan_build(kv_indptr, B, s_q, H, max_kv_len, ws, (hipStream_t)stream);
}

int dsa_mla_decode_csr_workspace_size(const dsa_mla_decode_csr_args* a, size_t* bytes) {
    if (!bytes) return DSA_ERR_NULL_POINTER;
    int ns, chunk;
    const int rc = validate_csr(a, &ns, &chunk);
    if (rc) return rc;
    *bytes = csr_ws_bytes(a, ns);
    return DSA_OK;
}
int dsa_mla_decode_csr(const dsa_mla_decode_csr_args* a, void* ws, size_t ws_bytes, void* stream) {
    int ns, chunk;
    const int rc = validate_csr(a, &ns, &chunk);
    if (rc) return rc;
    const size_t need = csr_ws_bytes(a, ns);
    if (need && (!ws || ws_bytes < need || ((uintptr_t)ws & 15))) return DSA_ERR_WORKSPACE;
    if (a->B == 0) return DSA_OK;
    hipStream_t st = (hipStream_t)stream;
    // uniform splits (no work plan) of few query rows or few heads: 32-head workgroups
    const bool narrow = ns >= 1 && narrow_path(a->kv_format, (int64_t)a->B * a->s_q, a->H, ns);
    FwdParams fp{};
    fp.H = a->H;
    fp.hgroups = narrow ? narrow_groups(a->H) : head_groups(a->H);
    fp.q = (const __bf16*)a->q;
    fp.q_sb = (int64_t)a->s_q * a->stride_q_b; fp.q_st = a->stride_q_b; fp.q_sh = a->stride_q_h;
    fp.kv = (const unsigned char*)a->kv;
    fp.kv_total_rows = a->total_tokens;
    fp.row_bytes = row_stride_bytes(a->kv_format, a->stride_kv_page);
    fp.block_size = 1;
    fp.seq_len_default = a->total_tokens;
    fp.kv_indptr = a->kv_indptr;
    fp.kv_indices = a->kv_indices;
    fp.out = (__bf16*)a->out;
    fp.o_sb = (int64_t)a->s_q * a->stride_o_b; fp.o_st = a->stride_o_b; fp.o_sh = a->stride_o_h;
    fp.lse = a->lse;
    fp.B = a->B; fp.s_q = a->s_q; fp.topk = a->max_kv_len; fp.chunk = chunk;
    fp.scale_log2 = a->softmax_scale * LOG2E;
    if (ns <= 0) return csr_plan_launch(fp, a->kv_format, a->max_kv_len, ws, ns == 0, st);
    if (ns > 1) {
        const size_t rows = (size_t)a->B * a->s_q * a->H;
        fp.part_o = (float*)ws;
        fp.part_lse = (float*)((char*)ws + (size_t)ns * rows * D_VO * sizeof(float));
    }
    int r = launch_fwd(fp, a->kv_format, a->B, a->s_q, ns, st, narrow);
    if (r || ns == 1) return r;
    return launch_combine(fp.part_o, fp.part_lse, ns, a->B * a->s_q, a->H, a->s_q, a->out, fp.o_sb, fp.o_st,
                          fp.o_sh, a->lse, st);
}
int dsa_mla_decode_mxfp8_workspace_size(const dsa_mla_decode_mxfp8_args* a, size_t* bytes) {
    if (!bytes) return DSA_ERR_NULL_POINTER;
    int ns, chunk;
    const int rc = validate_mx(a, &ns, &chunk);
    if (rc) return rc;
    *bytes = mx_ws_bytes(a, ns);
    return DSA_OK;
}
int dsa_mla_decode_mxfp8(const dsa_mla_decode_mxfp8_args* a, void* ws, size_t ws_bytes, void* stream) {
    int ns, chunk;
    const int rc = validate_mx(a, &ns, &chunk);
    if (rc) return rc;
    const size_t need = mx_ws_bytes(a, ns);
    if (need && (!ws || ws_bytes < need || ((uintptr_t)ws & 15))) return DSA_ERR_WORKSPACE;
    if (a->B == 0) return DSA_OK;
    hipStream_t st = (hipStream_t)stream;
    FwdParams fp{};
    fp.H = a->H;
    fp.hgroups = head_groups(a->H);
    const int64_t sq = a->s_q;
    fp.q = (const __bf16*)a->q_rope;
    fp.q_sb = sq * a->stride_q_rope_b; fp.q_st = a->stride_q_rope_b; fp.q_sh = a->stride_q_rope_h;
    fp.q8 = (const unsigned char*)a->q_nope;
    fp.q8_sb = sq * a->stride_q_nope_b; fp.q8_st = a->stride_q_nope_b; fp.q8_sh = a->stride_q_nope_h;
    fp.qsc = (const unsigned char*)a->q_scale;
    fp.qsc_sb = sq * a->stride_q_scale_b; fp.qsc_st = a->stride_q_scale_b; fp.qsc_sh = a->stride_q_scale_h;
    fp.kv = (const unsigned char*)a->kv_nope;
    fp.kv_sc = (const unsigned char*)a->kv_scale;
    fp.kv_ro = (const unsigned char*)a->kv_rope;
    fp.kvn_st = (uint32_t)a->stride_kv_nope_page;
    fp.kvs_st = (uint32_t)a->stride_kv_scale_page;
    fp.kvr_st = (uint32_t)a->stride_kv_rope_page * 2u;
    fp.kv_total_rows = a->total_tokens;
    fp.block_size = 1;
    fp.seq_len_default = a->total_tokens;
    fp.kv_indptr = a->kv_indptr;
    fp.kv_indices = a->kv_indices;
    fp.out = (__bf16*)a->out;
    fp.o_sb = sq * a->stride_o_b; fp.o_st = a->stride_o_b; fp.o_sh = a->stride_o_h;
    fp.lse = a->lse;
    fp.B = a->B; fp.s_q = a->s_q; fp.topk = a->max_kv_len; fp.chunk = chunk;
    fp.scale_log2 = a->softmax_scale * LOG2E;
    if (ns <= 0) return csr_plan_launch(fp, DSA_KV_MXFP8, a->max_kv_len, ws, ns == 0, st);
    if (ns > 1) {
        const size_t rows = (size_t)a->B * a->s_q * a->H;
        fp.part_o = (float*)ws;
        fp.part_lse = (float*)((char*)ws + (size_t)ns * rows * D_VO * sizeof(float));
    }
    int r = launch_fwd(fp, DSA_KV_MXFP8, a->B, a->s_q, ns, st);
    if (r || ns == 1) return r;
    return launch_combine(fp.part_o, fp.part_lse, ns, a->B * a->s_q, a->H, a->s_q, a->out, fp.o_sb, fp.o_st,
                          fp.o_sh, a->lse, st);
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
    if (!bytes) return DSA_ERR_NULL_POINTER;
    int ns;
    const int rc = validate_prefill(a, &ns);
    if (rc) return rc;
    *bytes = prefill_ws_bytes(ns, a->N, a->H);
    return DSA_OK;
}

int dsa_mla_prefill(const dsa_mla_prefill_args* a, void* ws, size_t ws_bytes, void* stream) {
    int ns;
    const int rc = validate_prefill(a, &ns);
    if (rc) return rc;
    const size_t need = prefill_ws_bytes(ns, a->N, a->H);
    if (need && (!ws || ws_bytes < need || ((uintptr_t)ws & 15))) return DSA_ERR_WORKSPACE;
    if (a->N == 0) return DSA_OK;
    bool narrow;
    prefill_plan(a->kv_format, a->N, a->H, a->num_splits, a->topk, &narrow);
    FwdParams fp{};
    fp.H = a->H;
    fp.hgroups = narrow ? narrow_groups(a->H) : head_groups(a->H);
    fp.q = (const __bf16*)a->q;
    fp.q_sb = a->q_stride_n; fp.q_st = 0; fp.q_sh = a->q_stride_h;
    fp.kv = (const unsigned char*)a->kv;
    fp.kv_total_rows = a->kv_rows;
    fp.row_bytes = row_stride_bytes(a->kv_format, a->kv_stride_row);
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
    fp.B = a->N; fp.s_q = 1; fp.topk = a->topk;
    fp.chunk = a->topk == 0 ? 0 : (a->topk + ns - 1) / ns;
    fp.causal = a->causal ? 2 : 0;
    fp.causal_offset = a->causal_offset;
    fp.reverse = 1;
    fp.scale_log2 = a->sm_scale * LOG2E;
    return prefill_launch(fp, a->kv_format, ns, nullptr, ws, (hipStream_t)stream, narrow);
}

int dsa_mla_prefill_v4_workspace_size(const dsa_mla_prefill_v4_args* a, size_t* bytes) {
    if (!bytes) return DSA_ERR_NULL_POINTER;
    int ns;
    const int rc = validate_v4(a, &ns);
    if (rc) return rc;
    *bytes = prefill_ws_bytes(ns, a->N, a->H);
    return DSA_OK;
}

int dsa_mla_prefill_v4(const dsa_mla_prefill_v4_args* a, void* ws, size_t ws_bytes, void* stream) {
    int ns;
    const int rc = validate_v4(a, &ns);
    if (rc) return rc;
    const size_t need = prefill_ws_bytes(ns, a->N, a->H);
    if (need && (!ws || ws_bytes < need || ((uintptr_t)ws & 15))) return DSA_ERR_WORKSPACE;
    if (a->N == 0) return DSA_OK;
    bool narrow;
    prefill_plan(DSA_KV_BF16_D512, a->N, a->H, a->num_splits, a->max_rows, &narrow);
    FwdParams fp{};
    fp.H = a->H;
    fp.hgroups = narrow ? narrow_groups(a->H) : head_groups(a->H);
    fp.q = (const __bf16*)a->q;
    fp.q_sb = a->stride_qo_n; fp.q_st = 0; fp.q_sh = a->stride_qo_h;
    fp.kv = (const unsigned char*)a->unified_kv;
    fp.kv_total_rows = a->total_pages;
    fp.kv2 = (const unsigned char*)a->kv;
    fp.kv2_rows = a->total_tokens;
    fp.row_bytes = (int64_t)a->stride_kv_page * 2;
    fp.block_size = 1;
    fp.ind_pre = a->kv_indptr_prefix; fp.idx_pre = a->kv_indices_prefix;
    fp.ind_ext = a->kv_indptr_extend; fp.idx_ext = a->kv_indices_extend;
    fp.out = (__bf16*)a->out;
    fp.o_sb = a->stride_qo_n; fp.o_st = 0; fp.o_sh = a->stride_qo_h;
    fp.lse = a->lse;
    fp.B = a->N; fp.s_q = 1; fp.topk = a->max_rows; fp.chunk = a->max_rows;
    fp.scale_log2 = a->softmax_scale * LOG2E;
    return prefill_launch(fp, DSA_KV_BF16_D512, ns, a->attn_sink, ws, (hipStream_t)stream, narrow);
}

int dsa_mla_prefill_v4_fp8_workspace_size(const dsa_mla_prefill_v4_fp8_args* a, size_t* bytes) {
    if (!bytes) return DSA_ERR_NULL_POINTER;
    int ns;
    const int rc = validate_v4fp8(a, &ns);
    if (rc) return rc;
    *bytes = prefill_ws_bytes(ns, a->N, a->H);
    return DSA_OK;
}

int dsa_mla_prefill_v4_fp8(const dsa_mla_prefill_v4_fp8_args* a, void* ws, size_t ws_bytes, void* stream) {
    int ns;
    const int rc = validate_v4fp8(a, &ns);
    if (rc) return rc;
    const size_t need = prefill_ws_bytes(ns, a->N, a->H);
    if (need && (!ws || ws_bytes < need || ((uintptr_t)ws & 15))) return DSA_ERR_WORKSPACE;
    if (a->N == 0) return DSA_OK;
    FwdParams fp{};
    fp.H = a->H;
    fp.hgroups = head_groups(a->H);
    fp.q = (const __bf16*)a->q_rope;
    fp.q_sb = a->stride_q_rope_n; fp.q_st = 0; fp.q_sh = a->stride_q_rope_h;
    fp.q8 = (const unsigned char*)a->q_nope;
    fp.q8_sb = a->stride_q_nope_n; fp.q8_st = 0; fp.q8_sh = a->stride_q_nope_h;
    // the 14 scales of a Q head follow its 448 codes in the same stream row
    fp.qsc = (const unsigned char*)a->q_nope + DSA_MLA_V4_NOPE;
    fp.qsc_sb = fp.q8_sb; fp.qsc_st = 0; fp.qsc_sh = fp.q8_sh;
    fp.kv = (const unsigned char*)a->unified_kv_nope;
    fp.kv_ro = (const unsigned char*)a->unified_kv_rope;
    fp.kv_total_rows = a->total_pages;
    fp.kv2 = (const unsigned char*)a->kv_nope;
    fp.kv2_ro = (const unsigned char*)a->kv_rope;
    fp.kv2_rows = a->total_tokens;
    fp.kvn_st = (uint32_t)a->stride_kv_nope_page;
    fp.kvr_st = (uint32_t)a->stride_kv_rope_page * 2u;
    fp.block_size = 1;
    fp.ind_pre = a->kv_indptr_prefix; fp.idx_pre = a->kv_indices_prefix;
    fp.ind_ext = a->kv_indptr_extend; fp.idx_ext = a->kv_indices_extend;
    fp.out = (__bf16*)a->out;
    fp.o_sb = a->stride_o_n; fp.o_st = 0; fp.o_sh = a->stride_o_h;
    fp.lse = a->lse;
    fp.B = a->N; fp.s_q = 1; fp.topk = a->max_rows; fp.chunk = a->max_rows;
    fp.scale_log2 = a->softmax_scale * LOG2E;
    return prefill_launch(fp, DSA_KV_MXFP8_V4, ns, a->attn_sink, ws, (hipStream_t)stream);
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
