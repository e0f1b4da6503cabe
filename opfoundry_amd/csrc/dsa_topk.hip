// DSA top-k index selection for gfx950: the step in front of the sparse-MLA
// kernels that turns one row of index scores per query token into the
// `indices` row those kernels gather (positions ascending, -1 padded).
//
// The reference leaves this step to its caller: "top-k semantics should
// already be reflected in kv_indices" (opus_attn/dsa_v4/README.md:185;
// opus_attn/dsa_v32/README.md:99).  The contract here is therefore this
// library's own and is spelled out in include/dsa_topk.h.
//
// Design.  One workgroup of 1024 threads (16 waves) per query token; a
// token's row is 4 B per position, so the path is HBM-bound byte work and
// uses no MFMA.  Each fp32 score maps to an order-preserving uint32 key
// (NaN highest, -0 == +0).  A radix select finds the k-th key: one pass
// histograms the top 12 key bits of every valid position into LDS, and the
// bin holding the k-th key is found with a workgroup scan.
// - Two-read path (k <= 4096 and <= 4096 keys in that bin): one ordered pass
//   stores the positions above the bin and the bin's (key, position) pairs in
//   LDS; the rest of the key is resolved over the candidates, and the two
//   ascending lists are merged into the output (select_in_lds).
// - Otherwise, 10-bit passes over the row refine the threshold until the k-th
//   key is resolved (at most two), and a last pass compacts the selected
//   positions in index order: every key above the threshold, plus the first
//   r positions whose key equals it (r = what the higher keys leave of k).
// Loads are 16-byte vector loads of four positions per lane, coalesced
// across the wave; the passes after the first hit the L2 / MALL.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dsa_topk.h"

namespace {

constexpr int TK_THREADS = 1024;
constexpr int TK_WAVES = TK_THREADS / 64;
constexpr int TK_FIRST_BITS = 12;          // first histogram: 4096 bins
constexpr int TK_NEXT_BITS = 10;           // refinement passes: 1024 bins
constexpr int TK_UNROLL = 8;               // float4 loads in flight per lane in a histogram pass
constexpr int TK_GROUP = 4;                // compaction: segments of 4096 positions loaded together
constexpr int TK_FAST_K = 4096;            // two-read path: top-k sizes whose positions LDS holds
constexpr int TK_CAND = 4096;              // two-read path: threshold-bin candidates LDS holds

// Order-preserving key: a > b as scores <=> key(a) > key(b) as uint32.  Every
// NaN maps to the largest key, and -0 to the key of +0.
__device__ __forceinline__ uint32_t order_key(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t mag = b & 0x7fffffffu;
    if (mag > 0x7f800000u) return 0xffffffffu;
    if (mag == 0) return 0x80000000u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The key's top L bits (L in {0, 12, 22, 32}).
__device__ __forceinline__ uint32_t key_top(uint32_t key, int L) {
    return L == 0 ? 0u : (L == 32 ? key : key >> (32 - L));
}

// Keys in the bins above this thread's: the workgroup total minus the inclusive scan.
__device__ __forceinline__ uint32_t tot_minus(uint32_t incl, uint32_t tot) { return tot - incl; }

// Number of entries of the ascending list a[0, n) below x.
__device__ __forceinline__ uint32_t count_below(const uint32_t* a, uint32_t n, uint32_t x) {
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (a[mid] < x) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Inclusive scan of one uint32 per thread over the workgroup; *total gets the
// workgroup's sum.  All threads must call it (it holds barriers).
__device__ __forceinline__ uint32_t wg_scan(uint32_t v, uint32_t* part, uint32_t* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t u = __shfl_up(v, d, 64);
        if (lane >= d) v += u;
    }
    if (lane == 63) part[w] = v;
    __syncthreads();
    if (w == 0) {
        uint32_t p = lane < TK_WAVES ? part[lane] : 0u;
#pragma unroll
        for (int d = 1; d < TK_WAVES; d <<= 1) {
            const uint32_t u = __shfl_up(p, d, 64);
            if (lane >= d) p += u;
        }
        if (lane < TK_WAVES) part[lane] = p;
    }
    __syncthreads();
    const uint32_t before = w ? part[w - 1] : 0u;
    *total = part[TK_WAVES - 1];
    __syncthreads();
    return v + before;
}

// Two-read path, after the 12-bit histogram has found the bin P holding the k-th
// key: `above` keys lie in higher bins and the r-th of the bin's cnt keys is the
// k-th overall.  One ordered pass over the row stores the above-bin positions and
// the bin's (key, position) pairs in LDS, both ascending; the remaining 20 key bits
// are resolved over the candidates alone, the r chosen candidates are compacted in
// position order, and the two ascending lists are merged into the output.
__device__ __forceinline__ void select_in_lds(const float4* __restrict__ row, int n, int n4, int k, uint32_t P,
                                              uint32_t above, uint32_t r, uint32_t cnt, uint32_t* hist,
                                              uint32_t* above_pos, uint2* cand, uint32_t* part,
                                              uint32_t* found, int32_t* __restrict__ out) {
    const int tid = threadIdx.x;
    uint32_t run_gt = 0, run_eq = 0;
    for (int base = 0; base < n4; base += TK_THREADS) {
        const int i = base + tid;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < n4) v = row[i];
        const float e[4] = {v.x, v.y, v.z, v.w};
        uint32_t keys[4], flags = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            keys[c] = order_key(e[c]);
            if (i >= n4 || 4 * i + c >= n) continue;
            const uint32_t top = keys[c] >> (32 - TK_FIRST_BITS);
            if (top > P) flags |= 1u << c;
            else if (top == P) flags |= 16u << c;
        }
        const uint32_t mine = (uint32_t)__builtin_popcount(flags & 15u) |
                              ((uint32_t)__builtin_popcount(flags >> 4) << 16);
        uint32_t tot;
        const uint32_t ex = wg_scan(mine, part, &tot) - mine;
        uint32_t gb = run_gt + (ex & 0xffffu), eb = run_eq + (ex >> 16);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if ((flags >> c) & 1u) {
                if (gb < (uint32_t)TK_FAST_K) above_pos[gb] = (uint32_t)(4 * i + c);
                ++gb;
            } else if ((flags >> (4 + c)) & 1u) {
                if (eb < (uint32_t)TK_CAND) cand[eb] = make_uint2(keys[c], (uint32_t)(4 * i + c));
                ++eb;
            }
        }
        run_gt += tot & 0xffffu;
        run_eq += tot >> 16;
    }
    __syncthreads();
    // the rest of the key (20 bits) over the candidates: two 10-bit digits
    uint32_t Pc = P;
    int L = TK_FIRST_BITS;
    bool take_all = false;
    uint32_t rr = r;
    for (int pass = 0; pass < 2; ++pass) {
        const int shift = 32 - L - TK_NEXT_BITS;
        hist[tid] = 0;  // 1024 bins, one per thread
        __syncthreads();
        for (uint32_t j = tid; j < cnt; j += TK_THREADS) {
            const uint32_t key = cand[j].x;
            if ((key >> (32 - L)) == Pc) atomicAdd(&hist[(key >> shift) & 1023u], 1u);
        }
        __syncthreads();
        const uint32_t c = hist[tid];
        uint32_t tot;
        const uint32_t acc = tot_minus(wg_scan(c, part, &tot), tot);
        if (acc < rr && acc + c >= rr) {
            found[0] = (uint32_t)tid;
            found[1] = acc;
            found[2] = c;
        }
        __syncthreads();
        const uint32_t digit = found[0], abv = found[1], cn = found[2];
        __syncthreads();
        rr -= abv;
        Pc = (Pc << TK_NEXT_BITS) | digit;
        L += TK_NEXT_BITS;
        if (rr == cn) {
            take_all = true;
            break;
        }
    }
    // the r chosen candidates, ascending, into hist[0, r)
    const uint32_t r_eff = take_all ? 0xffffffffu : rr;
    uint32_t cg = 0, ce = 0;
    for (uint32_t base = 0; base < cnt; base += TK_THREADS) {
        const uint32_t j = base + tid;
        uint32_t gt = 0, eq = 0;
        uint2 kp = make_uint2(0u, 0u);
        if (j < cnt) {
            kp = cand[j];
            const uint32_t top = key_top(kp.x, L);
            gt = top > Pc;
            eq = top == Pc;
        }
        const uint32_t mine = gt | (eq << 16);
        uint32_t tot;
        const uint32_t ex = wg_scan(mine, part, &tot) - mine;
        const uint32_t gb = cg + (ex & 0xffffu), eb = ce + (ex >> 16);
        if (gt) {
            const uint32_t slot = gb + (eb < r_eff ? eb : r_eff);
            if (slot < r) hist[slot] = kp.y;
        } else if (eq && eb < r_eff && gb + eb < r) {
            hist[gb + eb] = kp.y;
        }
        cg += tot & 0xffffu;
        ce += tot >> 16;
    }
    __syncthreads();
    // merge: an entry's slot is its rank in its own list plus the entries of the
    // other list below it (positions are distinct)
    for (uint32_t j = tid; j < above; j += TK_THREADS) {
        const uint32_t x = above_pos[j];
        const uint32_t slot = j + count_below(hist, r, x);
        if (slot < (uint32_t)k) out[slot] = (int32_t)x;
    }
    for (uint32_t j = tid; j < r; j += TK_THREADS) {
        const uint32_t y = hist[j];
        const uint32_t slot = j + count_below(above_pos, above, y);
        if (slot < (uint32_t)k) out[slot] = (int32_t)y;
    }
}

__global__ __launch_bounds__(TK_THREADS) void dsa_topk_kernel(
    const float* __restrict__ scores, int64_t score_stride, const int32_t* __restrict__ lengths,
    int32_t n_max, int32_t k, int32_t* __restrict__ indices, int64_t idx_stride) {
    __shared__ uint32_t hist[1 << TK_FIRST_BITS];  // histograms; then the chosen candidates
    __shared__ uint32_t above_pos[TK_FAST_K];        // two-read path: positions above the bin
    __shared__ uint2 cand[TK_CAND];                  // two-read path: (key, position) in the bin
    __shared__ uint32_t part[TK_WAVES];
    __shared__ uint32_t found[3];  // digit, keys above its bin, keys in its bin

    const int tid = threadIdx.x;
    const int64_t t = blockIdx.x;
    int n = lengths ? lengths[t] : n_max;
    n = n < 0 ? 0 : (n > n_max ? n_max : n);
    const float4* row = reinterpret_cast<const float4*>(scores + t * score_stride);
    int32_t* out = indices + t * idx_stride;
    const int n4 = (n + 3) >> 2;

    // Selection state: keys whose top L bits exceed P are taken; of those equal
    // to P, all are taken (take_all) or the first r in position order.
    uint32_t P = 0, r = (uint32_t)k;
    int L = 0;
    bool take_all = true;
    if (n > k) {
        take_all = false;
        for (int pass = 0; pass < 3; ++pass) {
            const int bits = pass == 0 ? TK_FIRST_BITS : TK_NEXT_BITS;
            const int nbins = 1 << bits;
            const int shift = 32 - L - bits;
            for (int b = tid; b < nbins; b += TK_THREADS) hist[b] = 0;
            __syncthreads();
            for (int i0 = tid; i0 < n4; i0 += TK_THREADS * TK_UNROLL) {
                float4 v[TK_UNROLL];
#pragma unroll
                for (int j = 0; j < TK_UNROLL; ++j) {
                    const int i = i0 + j * TK_THREADS;
                    if (i < n4) v[j] = row[i];
                }
#pragma unroll
                for (int j = 0; j < TK_UNROLL; ++j) {
                    const int i = i0 + j * TK_THREADS;
                    if (i >= n4) continue;
                    const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        if (4 * i + c >= n) continue;
                        const uint32_t key = order_key(e[c]);
                        if (key_top(key, L) == P) atomicAdd(&hist[(key >> shift) & (nbins - 1)], 1u);
                    }
                }
            }
            __syncthreads();
            // Thread tid owns bins [tid * per, tid * per + per); higher bins belong to
            // higher threads, so the keys above a thread's bins are total - inclusive.
            const int per = nbins / TK_THREADS;
            uint32_t s = 0;
            for (int j = 0; j < per; ++j) s += hist[tid * per + j];
            uint32_t tot;
            const uint32_t incl = wg_scan(s, part, &tot);
            uint32_t acc = tot - incl;
            for (int j = per - 1; j >= 0; --j) {
                const uint32_t c = hist[tid * per + j];
                if (acc < r && acc + c >= r) {  // exactly one bin in the workgroup holds the r-th key
                    found[0] = (uint32_t)(tid * per + j);
                    found[1] = acc;
                    found[2] = c;
                }
                acc += c;
            }
            __syncthreads();
            const uint32_t digit = found[0], above = found[1], cnt = found[2];
            __syncthreads();
            r -= above;
            P = (P << bits) | digit;
            L += bits;
            if (r == cnt) {
                take_all = true;
                break;
            }
            if (pass == 0 && k <= TK_FAST_K && cnt <= TK_CAND) {
                select_in_lds(row, n, n4, k, P, above, r, cnt, hist, above_pos, cand, part, found, out);
                return;  // uniform: every thread takes this branch
            }
        }
    }

    // Compaction in position order.  Per 4096 positions, one scan of packed
    // counts (above-threshold in the low half, equal in the high half; each is
    // at most 4096) gives every lane the counts of earlier positions.  An
    // equal-key position is taken iff fewer than r equal keys precede it; a
    // position's slot is the number of taken positions before it.
    const uint32_t r_eff = take_all ? 0xffffffffu : r;
    uint32_t run_gt = 0, run_eq = 0;
    // Segments of 4096 positions are loaded TK_GROUP at a time, and the next group's
    // loads are issued before this group's scans, so the scans' barriers overlap the
    // memory latency instead of waiting on one load each.
    float4 cur[TK_GROUP], nxt[TK_GROUP];
#pragma unroll
    for (int j = 0; j < TK_GROUP; ++j) {
        const int i = j * TK_THREADS + tid;
        if (i < n4) cur[j] = row[i];
    }
    for (int gbase = 0; gbase < n4; gbase += TK_GROUP * TK_THREADS) {
        const int gnext = gbase + TK_GROUP * TK_THREADS;
#pragma unroll
        for (int j = 0; j < TK_GROUP; ++j) {
            const int i = gnext + j * TK_THREADS + tid;
            if (i < n4) nxt[j] = row[i];
        }
#pragma unroll
        for (int j = 0; j < TK_GROUP; ++j) {
            const int sbase = gbase + j * TK_THREADS;
            if (sbase >= n4) break;  // uniform: the same for every thread
            const int i = sbase + tid;
            uint32_t flags = 0;      // bit c: above; bit 4 + c: equal
            if (i < n4) {
                const float e[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if (4 * i + c >= n) continue;
                    const uint32_t top = key_top(order_key(e[c]), L);
                    if (top > P) flags |= 1u << c;
                    else if (top == P) flags |= 16u << c;
                }
            }
            const uint32_t mine = (uint32_t)__builtin_popcount(flags & 15u) |
                                  ((uint32_t)__builtin_popcount(flags >> 4) << 16);
            uint32_t tot;
            const uint32_t ex = wg_scan(mine, part, &tot) - mine;
            uint32_t gb = run_gt + (ex & 0xffffu), eb = run_eq + (ex >> 16);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                // slots stay below k when the row is not modified during the call; the
                // bound check keeps a caller's race on `scores` from writing past the row
                if ((flags >> c) & 1u) {
                    const uint32_t slot = gb + (eb < r_eff ? eb : r_eff);
                    if (slot < (uint32_t)k) out[slot] = 4 * i + c;
                    ++gb;
                } else if ((flags >> (4 + c)) & 1u) {
                    if (eb < r_eff && gb + eb < (uint32_t)k) out[gb + eb] = 4 * i + c;
                    ++eb;
                }
            }
            run_gt += tot & 0xffffu;
            run_eq += tot >> 16;
        }
#pragma unroll
        for (int j = 0; j < TK_GROUP; ++j) cur[j] = nxt[j];
    }
    const uint32_t taken = run_gt + (run_eq < r_eff ? run_eq : r_eff);
    for (uint32_t j = taken + (uint32_t)tid; j < (uint32_t)k; j += TK_THREADS) out[j] = -1;
}

// ---------------------------------------------------------------------------
// Register-resident path for rows of at most TR_MAX_N positions (the decode
// shapes: 65536 positions and less).  The row is read from HBM once: lane
// tid keeps the keys of its TR_J 16-byte pieces (positions
// 4 (j * 1024 + tid) + c) in registers.  The first 12-bit histogram is built
// as the pieces land; the keys of the bin holding the k-th key go to an LDS
// list, and the two refinement digits are counted over that list alone.  The
// compaction in position order needs no second read: within a wave a
// position's rank comes from ballots, across waves and pieces from one table
// of per-(piece, wave) counts, scanned once.  The code is branch-free per
// key (selects, not conditional atomics).
// ---------------------------------------------------------------------------
constexpr int TR_J = 16;                                   // 16-byte pieces per lane
constexpr int TR_MAX_N = TK_THREADS * TR_J * 4;           // 65536 positions
constexpr int TR_CAND = 8192;                              // threshold-bin keys the LDS list holds
constexpr int TR_WAVE_LIST = 1536;                         // lists up to this long are refined by one wave

// order_key without branches (every case a select)
__device__ __forceinline__ uint32_t order_key_sel(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t mag = b & 0x7fffffffu;
    uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    k = mag == 0u ? 0x80000000u : k;
    return mag > 0x7f800000u ? 0xffffffffu : k;
}

// workgroup barrier over LDS only: outstanding global loads stay in flight
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
}

// Inclusive prefix sum over the 64 lanes of a wave: Hillis-Steele within each
// row of 16 lanes by DPP row shifts (a lane whose source lies outside its row
// adds 0), then the row totals by the row broadcasts of lanes 15 and 31.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
    return x;
}

__global__ __launch_bounds__(TK_THREADS) void dsa_topk_reg_kernel(
    const float* __restrict__ scores, int64_t score_stride, const int32_t* __restrict__ lengths,
    int32_t n_max, int32_t k, int32_t* __restrict__ indices, int64_t idx_stride) {
    __shared__ uint32_t hist[1 << TK_FIRST_BITS];
    __shared__ uint32_t cand[TR_CAND];
    __shared__ uint32_t part[TK_WAVES];
    __shared__ uint32_t found[4];  // digit, keys above its bin, keys in its bin; [3]: list fill
    __shared__ uint32_t sel[4];    // the threshold found by wave 0: P, L, r, take_all
    // per (piece j, wave w): keys above the threshold and keys equal to it;
    // then, in place, the counts of every (piece, wave) before it in position order
    __shared__ uint32_t tab_gt[TR_J * TK_WAVES], tab_eq[TR_J * TK_WAVES];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t t = blockIdx.x;
    int n = lengths ? lengths[t] : n_max;
    n = n < 0 ? 0 : (n > n_max ? n_max : n);
    const float4* row = reinterpret_cast<const float4*>(scores + t * score_stride);
    int32_t* out = indices + t * idx_stride;
    if (n == 0) {  // uniform
        for (int j = tid; j < k; j += TK_THREADS) out[j] = -1;
        return;
    }
    const int n4 = (n + 3) >> 2;

    // Pieces past the row re-read its last piece (in bounds) and are masked;
    // key 0 (below every valid key: the smallest, -inf, is 0x007fffff) marks a
    // position past the row.  Those land in bin 0, which holds no valid key and
    // so never holds the k-th (n > k valid keys lie above it).
    // The loads run TR_PF pieces ahead of the keys and the histogram, so that the
    // waves of a SIMD compute while later pieces are in flight (a wave that
    // issued all its loads at once would wait for the memory pipeline first).
    for (int b = tid; b < (1 << TK_FIRST_BITS); b += TK_THREADS) hist[b] = 0;
    if (tid == 0) found[3] = 0;
    lds_barrier();
    constexpr int TR_PF = 8;
    float4 v[TR_J];
#pragma unroll
    for (int j = 0; j < TR_PF; ++j) v[j] = row[min(j * TK_THREADS + tid, n4 - 1)];
    uint32_t key[TR_J][4];
#pragma unroll
    for (int j = 0; j < TR_J; ++j) {
        if (j + TR_PF < TR_J) v[j + TR_PF] = row[min((j + TR_PF) * TK_THREADS + tid, n4 - 1)];
        const int p0 = 4 * (j * TK_THREADS + tid);
        const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            // (a mask, not a select: the compiler turned the select into a branch
            // around the load of the piece's first value, waiting for every load)
            key[j][c] = order_key_sel(e[c]) & (0u - (uint32_t)(p0 + c < n));
            atomicAdd(&hist[key[j][c] >> (32 - TK_FIRST_BITS)], 1u);
        }
    }
    __syncthreads();

    // The threshold: keys in [t_lo, t_hi] are the tied ones (the first r of them
    // in position order are taken, or all), keys above t_hi are taken.
    uint32_t t_lo = 1u, t_hi = 0xffffffffu, r = (uint32_t)k;
    bool take_all = true;
    if (n > k) {
        take_all = false;
        constexpr int per = (1 << TK_FIRST_BITS) / TK_THREADS;
        uint32_t s = 0;
#pragma unroll
        for (int j = 0; j < per; ++j) s += hist[tid * per + j];
        uint32_t tot;
        uint32_t acc = tot_minus(wg_scan(s, part, &tot), tot);
#pragma unroll
        for (int j = per - 1; j >= 0; --j) {
            const uint32_t c = hist[tid * per + j];
            if (acc < r && acc + c >= r) {  // exactly one bin holds the r-th key
                found[0] = (uint32_t)(tid * per + j);
                found[1] = acc;
                found[2] = c;
            }
            acc += c;
        }
        __syncthreads();
        uint32_t P = found[0];
        const uint32_t cnt = found[2];
        r -= found[1];
        int L = TK_FIRST_BITS;
        __syncthreads();
        if (r == cnt) {
            take_all = true;
        } else if (cnt <= (uint32_t)TR_CAND) {
            // the bin's keys into the LDS list (any order): per-lane counts, a wave
            // scan, one list reservation per wave
            uint32_t mine = 0;
#pragma unroll
            for (int j = 0; j < TR_J; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c) mine += (key[j][c] >> (32 - TK_FIRST_BITS)) == P ? 1u : 0u;
            const uint32_t incl = wave_incl_scan(mine);
            uint32_t base = 0;
            if (lane == 63) base = atomicAdd(&found[3], incl);
            uint32_t pos = (uint32_t)__builtin_amdgcn_readlane((int)base, 63) + incl - mine;
#pragma unroll
            for (int j = 0; j < TR_J; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if ((key[j][c] >> (32 - TK_FIRST_BITS)) == P) cand[pos++] = key[j][c];
            // two 10-bit digits over the list: a short list by wave 0 alone (no
            // workgroup barrier per step; lane l owns bins 16 l .. 16 l + 15), a
            // long one by the workgroup
            __syncthreads();   // the list is complete
            if (cnt > (uint32_t)TR_WAVE_LIST) {
                for (int pass = 0; pass < 2; ++pass) {
                    const int shift = 32 - L - TK_NEXT_BITS;
                    hist[tid] = 0;  // 1024 bins, one per thread
                    __syncthreads();
                    for (uint32_t j = tid; j < cnt; j += TK_THREADS) {
                        const uint32_t kk = cand[j];
                        if ((kk >> (32 - L)) == P) atomicAdd(&hist[(kk >> shift) & 1023u], 1u);
                    }
                    __syncthreads();
                    const uint32_t c = hist[tid];
                    uint32_t tot2;
                    const uint32_t acc2 = tot_minus(wg_scan(c, part, &tot2), tot2);
                    if (acc2 < r && acc2 + c >= r) {
                        found[0] = (uint32_t)tid;
                        found[1] = acc2;
                        found[2] = c;
                    }
                    __syncthreads();
                    const uint32_t digit = found[0], abv = found[1], cn = found[2];
                    __syncthreads();
                    r -= abv;
                    P = (P << TK_NEXT_BITS) | digit;
                    L += TK_NEXT_BITS;
                    if (r == cn) {
                        take_all = true;
                        break;
                    }
                }
            } else {
                if (w == 0) {
                    for (int pass = 0; pass < 2; ++pass) {
                        const int shift = 32 - L - TK_NEXT_BITS;
#pragma unroll
                        for (int q = 0; q < 16; ++q) hist[64 * q + lane] = 0;
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        for (uint32_t j = lane; j < cnt; j += 64) {
                            const uint32_t kk = cand[j];
                            if ((kk >> (32 - L)) == P) atomicAdd(&hist[(kk >> shift) & 1023u], 1u);
                        }
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        uint32_t hb[16], sum = 0;
#pragma unroll
                        for (int q = 0; q < 16; ++q) {
                            hb[q] = hist[16 * lane + q];
                            sum += hb[q];
                        }
                        const uint32_t inc = wave_incl_scan(sum);
                        const uint32_t all = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
                        uint32_t acc2 = all - inc;   // keys in the bins of higher lanes
                        int hit = -1;
                        uint32_t h_abv = 0, h_cnt = 0;
#pragma unroll
                        for (int q = 15; q >= 0; --q) {
                            if (acc2 < r && acc2 + hb[q] >= r) {  // one bin of the wave holds the r-th key
                                hit = 16 * lane + q;
                                h_abv = acc2;
                                h_cnt = hb[q];
                            }
                            acc2 += hb[q];
                        }
                        const int src = __builtin_ctzll(__ballot(hit >= 0));
                        const uint32_t digit = (uint32_t)__builtin_amdgcn_readlane(hit, src);
                        r -= (uint32_t)__builtin_amdgcn_readlane((int)h_abv, src);
                        const uint32_t cn = (uint32_t)__builtin_amdgcn_readlane((int)h_cnt, src);
                        P = (P << TK_NEXT_BITS) | digit;
                        L += TK_NEXT_BITS;
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // bins read before the next clear
                        if (r == cn) {
                            take_all = true;
                            break;
                        }
                    }
                    if (lane == 0) {
                        sel[0] = P;
                        sel[1] = (uint32_t)L;
                        sel[2] = r;
                        sel[3] = take_all ? 1u : 0u;
                    }
                }
                __syncthreads();
                P = sel[0];
                L = (int)sel[1];
                r = sel[2];
                take_all = sel[3] != 0u;
            }
        } else {
            // more tied keys than the list holds: the two digits over the registers;
            // a key outside the prefix counts in a bin of its lane's own (no two lanes
            // of a wave share it), so the code stays free of branches
            for (int pass = 0; pass < 2; ++pass) {
                const int shift = 32 - L - TK_NEXT_BITS;
                hist[tid] = 0;
                if (tid < 64) hist[1024 + tid] = 0;
                __syncthreads();
#pragma unroll
                for (int j = 0; j < TR_J; ++j)
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const uint32_t kk = key[j][c];
                        const bool in = (kk >> (32 - L)) == P;
                        atomicAdd(&hist[in ? (kk >> shift) & 1023u : 1024u + lane], 1u);
                    }
                __syncthreads();
                const uint32_t c = hist[tid];
                uint32_t tot2;
                const uint32_t acc2 = tot_minus(wg_scan(c, part, &tot2), tot2);
                if (acc2 < r && acc2 + c >= r) {
                    found[0] = (uint32_t)tid;
                    found[1] = acc2;
                    found[2] = c;
                }
                __syncthreads();
                const uint32_t digit = found[0], abv = found[1], cn = found[2];
                __syncthreads();
                r -= abv;
                P = (P << TK_NEXT_BITS) | digit;
                L += TK_NEXT_BITS;
                if (r == cn) {
                    take_all = true;
                    break;
                }
            }
        }
        t_lo = L == 32 ? P : P << (32 - L);
        t_hi = L == 32 ? P : t_lo | ((1u << (32 - L)) - 1u);
    }

    // Compaction.  Position order is (piece j, wave, lane, c).  Per lane and
    // piece, the counts of above and tied keys (0..4) are packed ten bits
    // apart, three to a word, and scanned over the wave with DPP (a wave
    // prefix is at most 256); the per-(piece, wave) totals, scanned once over
    // the workgroup, give the counts of everything earlier.  The output is
    // staged in LDS (the candidate list is free by now) and leaves in
    // coalesced rows when it fits there.
    const uint32_t r_eff = take_all ? 0xffffffffu : r;
    constexpr int NW = (2 * TR_J + 2) / 3;   // count words
    uint32_t fl4[TR_J / 4] = {};             // flags of pieces 4q..4q+3: bit c above, 4 + c tied
    uint32_t cw[NW] = {};
#pragma unroll
    for (int j = 0; j < TR_J; ++j) {
        uint32_t f = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t kk = key[j][c];
            f |= (kk > t_hi ? 1u : 0u) << c;
            f |= (kk >= t_lo && kk <= t_hi ? 16u : 0u) << c;
        }
        fl4[j >> 2] |= f << (8 * (j & 3));
        cw[(2 * j) / 3] += (uint32_t)__builtin_popcount(f & 15u) << (10 * ((2 * j) % 3));
        cw[(2 * j + 1) / 3] += (uint32_t)__builtin_popcount(f >> 4) << (10 * ((2 * j + 1) % 3));
    }
    uint32_t ex[NW];   // exclusive wave prefixes of the packed counts
#pragma unroll
    for (int q = 0; q < NW; ++q) {
        const uint32_t inc = wave_incl_scan(cw[q]);
        ex[q] = inc - cw[q];
        const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
        if (lane == 0) {
#pragma unroll
            for (int f3 = 0; f3 < 3; ++f3) {
                const int fi = 3 * q + f3;   // field: 2j above, 2j + 1 tied
                if (fi < 2 * TR_J) {
                    const uint32_t v10 = (tot >> (10 * f3)) & 1023u;
                    if (fi & 1) tab_eq[(fi >> 1) * TK_WAVES + w] = v10;
                    else tab_gt[(fi >> 1) * TK_WAVES + w] = v10;
                }
            }
        }
    }
    __syncthreads();
    // exclusive scan of the TR_J * TK_WAVES = 256 (piece, wave) totals, in
    // position order, by the first four waves
    static_assert(TR_J * TK_WAVES == 4 * 64, "one table entry per lane of waves 0..3");
    uint32_t xg = 0, xe = 0;
    if (w < 4) {
        xg = wave_incl_scan(tab_gt[tid]);
        xe = wave_incl_scan(tab_eq[tid]);
        if (lane == 63) {
            part[2 * w] = xg;
            part[2 * w + 1] = xe;
        }
    }
    __syncthreads();
    if (w < 4) {
        uint32_t bg = 0, be = 0;
        for (int u = 0; u < w; ++u) {
            bg += part[2 * u];
            be += part[2 * u + 1];
        }
        // inclusive -> exclusive: less this entry's own totals
        tab_gt[tid] = bg + xg - tab_gt[tid];
        tab_eq[tid] = be + xe - tab_eq[tid];
    }
    __syncthreads();
    const bool staged = k <= TR_CAND;   // uniform
    // (positions recomputed from an opaque copy of tid: kept from the loads
    // above, the compiler spills them)
    int tq = tid;
    asm volatile("" : "+v"(tq));
    // slots by selects, one masked store per position: an above key takes slot
    // (above before it) + min(tied before it, r); a tied key is taken iff fewer
    // than r tied keys precede it.  Slots stay below k when the row is not
    // modified during the call; the bound check keeps a caller's race on
    // `scores` from writing past the row.
    auto emit = [&](auto&& store) {
#pragma unroll
        for (int j = 0; j < TR_J; ++j) {
            uint32_t gb = tab_gt[j * TK_WAVES + w] + ((ex[(2 * j) / 3] >> (10 * ((2 * j) % 3))) & 1023u);
            uint32_t eb = tab_eq[j * TK_WAVES + w] + ((ex[(2 * j + 1) / 3] >> (10 * ((2 * j + 1) % 3))) & 1023u);
            const int i = j * TK_THREADS + tq;
            const uint32_t f = (fl4[j >> 2] >> (8 * (j & 3))) & 0xffu;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                // (arithmetic, not nested selects: those the compiler turns into branches)
                const uint32_t a = (f >> c) & 1u, e = (f >> (4 + c)) & 1u;
                const uint32_t over = max(eb, r_eff) - r_eff;        // tied keys before it past r
                const uint32_t ok = a | (e & (uint32_t)(eb < r_eff));
                const uint32_t slot = (gb + eb - a * over) | (ok - 1u);   // not taken: 0xffffffff
                gb += a;
                eb += e;
                if (slot < (uint32_t)k) store(slot, 4 * i + c);
            }
        }
    };
    if (staged) emit([&](uint32_t sl, int v) { cand[sl] = (uint32_t)v; });
    else emit([&](uint32_t sl, int v) { out[sl] = v; });
    // the slots past the taken positions: -1
    const uint32_t all_g = part[0] + part[2] + part[4] + part[6];
    const uint32_t all_e = part[1] + part[3] + part[5] + part[7];
    const uint32_t taken = all_g + (all_e < r_eff ? all_e : r_eff);
    if (staged) {
        for (uint32_t j = taken + (uint32_t)tid; j < (uint32_t)k; j += TK_THREADS) cand[j] = 0xffffffffu;
        __syncthreads();
        for (int j = tid; j < k; j += TK_THREADS) out[j] = (int32_t)cand[j];
    } else {
        for (uint32_t j = taken + (uint32_t)tid; j < (uint32_t)k; j += TK_THREADS) out[j] = -1;
    }
}

}  // namespace

extern "C" {

int dsa_topk_indices(const float* scores, int64_t score_stride, const int32_t* lengths, int32_t n_tokens,
                     int32_t n_max, int32_t topk, int32_t* indices, int64_t idx_stride, void* stream) {
    if (n_tokens < 0 || n_max < 0 || topk < 0 || n_max > DSA_TOPK_MAX_N) return DSA_ERR_BAD_SHAPE;
    if (n_tokens == 0 || topk == 0) return DSA_OK;
    if (!indices || (n_max > 0 && !scores)) return DSA_ERR_NULL_POINTER;
    if (idx_stride < topk || score_stride < n_max) return DSA_ERR_BAD_SHAPE;
    if ((score_stride % 4) || ((uintptr_t)scores & 15) || ((uintptr_t)indices & 3)) return DSA_ERR_BAD_STRIDE;
    if (n_max <= TR_MAX_N)
        hipLaunchKernelGGL(dsa_topk_reg_kernel, dim3((unsigned)n_tokens), dim3(TK_THREADS), 0, (hipStream_t)stream,
                           scores, score_stride, lengths, n_max, topk, indices, idx_stride);
    else
        hipLaunchKernelGGL(dsa_topk_kernel, dim3((unsigned)n_tokens), dim3(TK_THREADS), 0, (hipStream_t)stream,
                           scores, score_stride, lengths, n_max, topk, indices, idx_stride);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

}  // extern "C"
