// Shared device and host helpers for the gfx950 decode hot path.
//
// Everything here is written for CDNA4 wave64: 64-lane wavefronts, DPP
// row operations for intra-row (16-lane) reductions, v_dot4_i32_i8 for the
// int8 dot products, and 16-byte global loads for weight streaming.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "taraference_hip.h"

#define TF_WAVE 64

// ---------------------------------------------------------------- numerics

// Exact binary16 -> binary32 (v_cvt_f32_f16; exact for every input).
__device__ __forceinline__ float tf_h2f(uint32_t h16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(h16 & 0xffffu));
    return (float)h;
}

// Four signed int8 products accumulated into c (v_dot4_i32_i8).
__device__ __forceinline__ int tf_dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// ------------------------------------------------------ wave64 reductions

// DPP controls (GFX9 encoding).
#define TF_DPP_QUAD_1032 0xB1   // quad_perm [1,0,3,2]  (xor 1)
#define TF_DPP_QUAD_2301 0x4E   // quad_perm [2,3,0,1]  (xor 2)
#define TF_DPP_ROW_HALF_MIRROR 0x141
#define TF_DPP_ROW_MIRROR 0x140

template <int CTRL>
__device__ __forceinline__ float tf_dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                           0xF, 0xF, false));
}

// Sum over each 16-lane row; every lane of the row receives the row sum.
__device__ __forceinline__ float tf_row16_sum(float v) {
    v += tf_dpp<TF_DPP_QUAD_1032>(v);
    v += tf_dpp<TF_DPP_QUAD_2301>(v);
    v += tf_dpp<TF_DPP_ROW_HALF_MIRROR>(v);
    v += tf_dpp<TF_DPP_ROW_MIRROR>(v);
    return v;
}

// Sum over aligned groups of LANES lanes (16, 32 or 64); every lane of the
// group receives the group sum.
template <int LANES>
__device__ __forceinline__ float tf_group_sum(float v) {
    static_assert(LANES == 16 || LANES == 32 || LANES == 64, "group size");
    v = tf_row16_sum(v);
    if (LANES >= 32) v += __shfl_xor(v, 16, 64);
    if (LANES >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ float tf_group32_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 1, 64));
    v = fmaxf(v, __shfl_xor(v, 2, 64));
    v = fmaxf(v, __shfl_xor(v, 4, 64));
    v = fmaxf(v, __shfl_xor(v, 8, 64));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return v;
}

// ---------------------------------------------------------- vector loads

typedef uint32_t tf_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t tf_u32x2 __attribute__((ext_vector_type(2)));
// 16-byte / 8-byte loads from addresses that are only 4-byte aligned
// (212-byte Q6_K blocks).  gfx950 global_load_dwordx4 needs dword alignment.
struct __attribute__((packed, aligned(4))) tf_a4x4 { tf_u32x4 v; };
struct __attribute__((packed, aligned(4))) tf_a4x2 { tf_u32x2 v; };

__device__ __forceinline__ tf_u32x4 tf_ld16(const void* p) {
    return reinterpret_cast<const tf_u32x4*>(p)[0];
}
__device__ __forceinline__ tf_u32x4 tf_ld16_a4(const void* p) {
    return reinterpret_cast<const tf_a4x4*>(p)->v;
}
__device__ __forceinline__ tf_u32x2 tf_ld8_a4(const void* p) {
    return reinterpret_cast<const tf_a4x2*>(p)->v;
}

// ---------------------------------------------------------------- Q8 math

// One value of the Q8 activation format used by the reference
// (kernels/gemv.cu:36-37): q = amax == 0 ? 0 : rint_even(x / d) with
// d = amax * fl(1/127) and an IEEE-correct division.
__device__ __forceinline__ int tf_q8_value(float x, float amax, float d) {
    return amax == 0.f ? 0 : (int)__builtin_rintf(x / d);
}

// f32 -> f16 bits, truncating the mantissa and adding one ulp when the first
// dropped bit is set (kernels/common.cu:9-38); subnormals, zero, inf and nan
// as the reference.
__device__ __forceinline__ uint16_t tf_f2h_halfup(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t absx = x & 0x7fffffffu;
    if (absx == 0u) return (uint16_t)sign;
    if (absx >= 0x7f800000u) return (uint16_t)(sign | (absx == 0x7f800000u ? 0x7c00u : 0x7e00u));
    if (absx < 0x33000000u) return (uint16_t)sign;
    if (absx >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);
    const int e = (int)((absx >> 23) & 0xff) - 127 + 15;
    uint32_t mant = absx & 0x7fffffu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t hm = mant >> shift;
        if ((mant >> (shift - 1)) & 1u) hm += 1u;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    if (mant & 0x1000u) h += 1u;
    return (uint16_t)(sign | h);
}

// ------------------------------------------------------------ host helpers



#define TF_CHECK_ARG(cond)                         \
    do {                                           \
        if (!(cond)) return (int)hipErrorInvalidValue; \
    } while (0)

#define TF_LAUNCH_RESULT() ((int)hipGetLastError())

static inline hipStream_t tf_stream(tf_stream_t s) {
    return reinterpret_cast<hipStream_t>(s);
}
