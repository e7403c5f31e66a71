// HBM -> LDS copies for gfx950 (global_load_lds_dwordx4) and the 16x16x32
// f16 matrix-core step, shared by the flash-decode partial and the
// persistent decode step's long-context attention.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 tf_h16x8 __attribute__((ext_vector_type(8)));
typedef float tf_f32x4v __attribute__((ext_vector_type(4)));

// One 1 KB copy: lane l moves the 16 bytes at src to LDS byte offset
// lds_off + 16 l (no register staging; the copy counts on the wave's vector
// memory counter and completes in issue order with its other vector memory
// operations).  The LDS base goes through M0, which the compiler also uses:
// it is saved and restored around the copy.  lds_off must be wave-uniform.
__device__ __forceinline__ void tf_lds_dma16(const void* src, uint32_t lds_off) {
    const uint32_t la = __builtin_amdgcn_readfirstlane(lds_off);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(la), "v"(src)
        : "memory");
}

// LDS byte offset of a pointer into LDS.
__device__ __forceinline__ uint32_t tf_lds_off(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// v_mfma_f32_16x16x32_f16: lane l supplies A[l % 16][8 g .. 8 g + 7] and
// B[8 g .. 8 g + 7][l % 16] (g = l / 16) and receives C[4 g + r][l % 16].
__device__ __forceinline__ tf_f32x4v tf_mfma_f16_k32(tf_h16x8 a, tf_h16x8 b, tf_f32x4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
