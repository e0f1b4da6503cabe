// dsa_lds.h - vector types, 32-bit LDS pointers, LDS-DMA loads and wait /
// barrier helpers shared by the gfx950 kernels of libdsa_mla.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

#define LDS_AS __attribute__((address_space(3)))

// 32-bit LDS addresses: every LDS access in the kernels goes through these
// (a generic pointer would cost a 64-bit VGPR pair per address).
typedef LDS_AS unsigned char* lds_ptr;
typedef const LDS_AS unsigned char* lds_cptr;

template <class V>
__device__ __forceinline__ V lds_ld(lds_cptr p) {
    return *reinterpret_cast<const LDS_AS V*>(p);
}

template <class V>
__device__ __forceinline__ void lds_st(lds_ptr p, V v) {
    *reinterpret_cast<LDS_AS V*>(p) = v;
}

__device__ __forceinline__ s16x4 lds_read_tr16(lds_cptr p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS s16x4*)(p));
}

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt left at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
}

// Opaque copy: stops the compiler from hoisting per-lane address math out of
// the tile loop (which would pin dozens of loop-invariant VGPRs).
__device__ __forceinline__ int opaque(int v) {
    asm("" : "+v"(v));
    return v;
}
// The same as volatile asm, which is never merged with another copy: values
// derived from it are computed where they are used, so a one-off epilogue does
// not keep a prologue value alive across the tile loop.
__device__ __forceinline__ int opaque_here(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// 16-byte LDS-DMA load: lane l's 16 bytes from gsrc land at lds_wave_base +
// 16*l.  Issued through inline asm so the compiler neither waits on it at the
// next LDS read nor folds it into its own vmcnt accounting: the tile loop
// tracks these loads with explicit s_waitcnt vmcnt(N), and no other vector
// memory load is issued inside the loop.
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

// The same load for a wave-uniform source row: 64-bit base in SGPRs plus a
// 32-bit per-lane byte offset (no per-lane 64-bit address arithmetic).
__device__ __forceinline__ void lds_dma16_s(const void* sbase, unsigned voff, lds_ptr lds_wave_base) {
    const unsigned m0v = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_wave_base);
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2"
        :
        : "s"(m0v), "v"(voff), "s"(sbase)
        : "memory", "m0");
}

// Workgroup barrier for the tile loop: LDS accesses of this wave complete,
// then s_barrier.  Unlike __syncthreads() it does not drain vector memory, so
// the LDS-DMA gathers of later tiles stay in flight across it.
__device__ __forceinline__ void tile_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
