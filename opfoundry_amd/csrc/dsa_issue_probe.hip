// dsa_issue_probe.hip - measurement probe, built as libdsa_issue_probe.so
// (not part of libdsa_mla.so and not a drop-in entry point).
//
// The forward kernels run one wave per SIMD (Q and the O accumulators fill the
// register file), so whatever a wave issues besides its MFMAs can only hide in
// the cycles its own MFMAs occupy the matrix pipe.  This probe measures how
// much of that happens for the instructions the 656-B tile loop issues:
//   mode 0  4 independent 32x32x16 f16 MFMAs per trip (AGPR accumulators bound
//           through inline asm, as the O accumulators are)
//   mode 1  mode 0 plus one dequant piece (mantissa extraction, 4
//           v_cvt_scalef32_pk_f16_fp8, 4 v_pk_mul_f16) after the 4 MFMAs
//   mode 2  the same piece split between the single MFMAs
//   mode 3  mode 2 plus the piece's ds_write_b128
//   mode 4  mode 0 plus 4 independent v_fma_f32 after every MFMA
//   mode 5  one dependent chain of 32x32x16 f16 MFMAs (operands in registers)
//   mode 6  four interleaved chains of the same MFMAs
//   mode 7  mode 0's 4 independent MFMAs as compiler builtins (VGPR
//           accumulators, the compiler's own wait states)
//   mode 8  mode 0 without the s_nop before each MFMA
// MFMA operands are small normal fp16 numbers, as the kernels' are.
// 256 workgroups of 256 threads (one wave per SIMD on every CU), `iters` trips
// of 4 MFMAs (modes 0-4) or 36-MFMA chains (modes 5, 6).  Each thread writes one
// float derived from every result, so no work is dead.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dsa_lds.h"

namespace {

__device__ __forceinline__ void mfma_a(f32x16& acc, u32x4 a, u32x4 b) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_a_nn(f32x16& acc, u32x4 a, u32x4 b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ unsigned opq(unsigned v) {
    asm volatile("" : "+v"(v));
    return v;
}
// one dequant piece of the 656-B loop: 8 codes times a per-128 fp32 scale
__device__ __forceinline__ u32x4 piece(unsigned c0, unsigned c1, unsigned s) {
    const float sc = __uint_as_float(s);
    const _Float16 m16 = (_Float16)__uint_as_float((s & 0x007FFFFFu) | 0x3F800000u);
    const f16x2 mm = {m16, m16};
    const f16x2 h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)c0, sc, false) * mm;
    const f16x2 h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)c0, sc, true) * mm;
    const f16x2 h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)c1, sc, false) * mm;
    const f16x2 h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)c1, sc, true) * mm;
    return u32x4{__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1), __builtin_bit_cast(unsigned, h2),
                 __builtin_bit_cast(unsigned, h3)};
}

template <int MODE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
dsa_issue_probe_kernel(float* __restrict__ out, int iters) {
    __shared__ u32x4 lds[4 * 256];
    const unsigned t = threadIdx.x;
    f32x16 o0 = {}, o1 = {}, o2 = {}, o3 = {};
    f32x16 ch[4] = {};
    const f16x8 ah = {(_Float16)(t & 7), 1, 2, 3, 4, 5, 6, 7}, bh = {1, 1, 1, 1, 1, 1, 1, (_Float16)(blockIdx.x & 7)};
    const u32x4 a = __builtin_bit_cast(u32x4, ah), b = __builtin_bit_cast(u32x4, bh);
    unsigned c0 = t * 0x01010101u ^ 0x38383838u, c1 = c0 ^ 0x01010101u;
    const unsigned s = 0x3c123456u;
    u32x4 acc = {};
    float f0 = (float)t * 0.00390625f, f1 = 0.5f, f2 = 0.25f, f3 = 0.125f;   // (the fma chains stay bounded)
    for (int i = 0; i < iters; ++i) {
        if constexpr (MODE == 0) {
            mfma_a(o0, a, b); mfma_a(o1, a, b); mfma_a(o2, a, b); mfma_a(o3, a, b);
        } else if constexpr (MODE == 7) {
            const f16x8 a8 = __builtin_bit_cast(f16x8, a), b8 = __builtin_bit_cast(f16x8, b);
            o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8, b8, o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8, b8, o1, 0, 0, 0);
            o2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8, b8, o2, 0, 0, 0);
            o3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8, b8, o3, 0, 0, 0);
        } else if constexpr (MODE == 8) {
            mfma_a_nn(o0, a, b); mfma_a_nn(o1, a, b); mfma_a_nn(o2, a, b); mfma_a_nn(o3, a, b);
        } else if constexpr (MODE == 1) {
            mfma_a(o0, a, b); mfma_a(o1, a, b); mfma_a(o2, a, b); mfma_a(o3, a, b);
            acc ^= piece(opq(c0), opq(c1), opq(s));
        } else if constexpr (MODE == 2 || MODE == 3) {
            const unsigned x0 = opq(c0), x1 = opq(c1), xs = opq(s);
            const float sc = __uint_as_float(xs);
            mfma_a(o0, a, b);
            const _Float16 m16 = (_Float16)__uint_as_float((xs & 0x007FFFFFu) | 0x3F800000u);
            const f16x2 mm = {m16, m16};
            f16x2 h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)x0, sc, false);
            __builtin_amdgcn_sched_barrier(0);
            mfma_a(o1, a, b);
            f16x2 h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)x0, sc, true);
            f16x2 h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)x1, sc, false);
            f16x2 h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)x1, sc, true);
            __builtin_amdgcn_sched_barrier(0);
            mfma_a(o2, a, b);
            h0 = h0 * mm; h1 = h1 * mm; h2 = h2 * mm; h3 = h3 * mm;
            __builtin_amdgcn_sched_barrier(0);
            const u32x4 r = {__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1),
                             __builtin_bit_cast(unsigned, h2), __builtin_bit_cast(unsigned, h3)};
            if constexpr (MODE == 3) lds[(t + 256u * (i & 3)) & 1023u] = r;
            else acc ^= r;
            __builtin_amdgcn_sched_barrier(0);
            mfma_a(o3, a, b);
            __builtin_amdgcn_sched_barrier(0);
        } else if constexpr (MODE == 4) {
#define DSA_PROBE_FMA4 f0 = __builtin_fmaf(f0, f1, f2); f1 = __builtin_fmaf(f1, f2, f3); \
                       f2 = __builtin_fmaf(f2, f3, f0); f3 = __builtin_fmaf(f3, f0, f1);
            mfma_a(o0, a, b); DSA_PROBE_FMA4 __builtin_amdgcn_sched_barrier(0);
            mfma_a(o1, a, b); DSA_PROBE_FMA4 __builtin_amdgcn_sched_barrier(0);
            mfma_a(o2, a, b); DSA_PROBE_FMA4 __builtin_amdgcn_sched_barrier(0);
            mfma_a(o3, a, b); DSA_PROBE_FMA4 __builtin_amdgcn_sched_barrier(0);
#undef DSA_PROBE_FMA4
        } else {
            constexpr int NCH = MODE == 5 ? 1 : 4;
#pragma unroll
            for (int k = 0; k < 36; k += NCH)
#pragma unroll
                for (int j = 0; j < NCH; ++j) ch[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, ch[j], 0, 0, 0);
        }
    }
    float r = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) r += o0[k] + o1[k] + o2[k] + o3[k] + ch[0][k] + ch[1][k] + ch[2][k] + ch[3][k];
    r += __uint_as_float(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) + f0 + f1 + f2 + f3;
    if constexpr (MODE == 3) {
        __syncthreads();
        r += __uint_as_float(lds[t][0]);
    }
    out[blockIdx.x * 256 + t] = r;
}

}  // namespace

// Launch one probe run: mode 0..8, `iters` trips, `out` a device buffer of
// 65536 floats, on `stream` (a hipStream_t; NULL = the null stream).  Returns
// 0, -2 for a mode or trip count out of range, -8 for a HIP error.
extern "C" int dsa_issue_probe(int mode, int iters, float* out, void* stream) {
    if (mode < 0 || mode > 8 || iters <= 0 || !out) return -2;
    const hipStream_t st = (hipStream_t)stream;
    const dim3 grid(256), block(256);
    switch (mode) {
        case 0: hipLaunchKernelGGL(dsa_issue_probe_kernel<0>, grid, block, 0, st, out, iters); break;
        case 1: hipLaunchKernelGGL(dsa_issue_probe_kernel<1>, grid, block, 0, st, out, iters); break;
        case 2: hipLaunchKernelGGL(dsa_issue_probe_kernel<2>, grid, block, 0, st, out, iters); break;
        case 3: hipLaunchKernelGGL(dsa_issue_probe_kernel<3>, grid, block, 0, st, out, iters); break;
        case 4: hipLaunchKernelGGL(dsa_issue_probe_kernel<4>, grid, block, 0, st, out, iters); break;
        case 5: hipLaunchKernelGGL(dsa_issue_probe_kernel<5>, grid, block, 0, st, out, iters); break;
        case 6: hipLaunchKernelGGL(dsa_issue_probe_kernel<6>, grid, block, 0, st, out, iters); break;
        case 7: hipLaunchKernelGGL(dsa_issue_probe_kernel<7>, grid, block, 0, st, out, iters); break;
        default: hipLaunchKernelGGL(dsa_issue_probe_kernel<8>, grid, block, 0, st, out, iters); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -8;
}
