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

}  // namespace

extern "C" {

int dsa_topk_indices(const float* scores, int64_t score_stride, const int32_t* lengths, int32_t n_tokens,
                     int32_t n_max, int32_t topk, int32_t* indices, int64_t idx_stride, void* stream) {
    if (n_tokens < 0 || n_max < 0 || topk < 0 || n_max > DSA_TOPK_MAX_N) return DSA_ERR_BAD_SHAPE;
    if (n_tokens == 0 || topk == 0) return DSA_OK;
    if (!indices || (n_max > 0 && !scores)) return DSA_ERR_NULL_POINTER;
    if (idx_stride < topk || score_stride < n_max) return DSA_ERR_BAD_SHAPE;
    if ((score_stride % 4) || ((uintptr_t)scores & 15) || ((uintptr_t)indices & 3)) return DSA_ERR_BAD_STRIDE;
    hipLaunchKernelGGL(dsa_topk_kernel, dim3((unsigned)n_tokens), dim3(TK_THREADS), 0, (hipStream_t)stream,
                       scores, score_stride, lengths, n_max, topk, indices, idx_stride);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_HIP;
}

}  // extern "C"
