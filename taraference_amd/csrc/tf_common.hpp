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
#define TF_DPP_ROW_ROR8 0x128   // row_ror:8 (lane i of a row reads lane i ^ 8)
#define TF_DPP_ROW_ROR4 0x124   // row_ror:4 (lane i reads lane (i - 4) mod 16)

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

// Value of lane (lane ^ 16): ds_swizzle bit mode, and 0x1F, xor 0x10.
__device__ __forceinline__ float tf_swap16(float v) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

__device__ __forceinline__ float tf_readlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over aligned groups of LANES lanes (16, 32 or 64); every lane of the
// group receives the group sum, added as ((r0 + r1) + (r2 + r3)) of the
// 16-lane row sums.
template <int LANES>
__device__ __forceinline__ float tf_group_sum(float v) {
    static_assert(LANES == 16 || LANES == 32 || LANES == 64, "group size");
    v = tf_row16_sum(v);
    if (LANES >= 32) v += tf_swap16(v);
    if (LANES >= 64) v = tf_readlane(v, 0) + tf_readlane(v, 32);
    return v;
}

template <int CTRL>
__device__ __forceinline__ int tf_dppi(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Maximum over each 16-lane row (DPP only); every lane receives it.
__device__ __forceinline__ float tf_row16_max(float v) {
    v = fmaxf(v, tf_dpp<TF_DPP_QUAD_1032>(v));
    v = fmaxf(v, tf_dpp<TF_DPP_QUAD_2301>(v));
    v = fmaxf(v, tf_dpp<TF_DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, tf_dpp<TF_DPP_ROW_MIRROR>(v));
    return v;
}

// The same for values >= 0 (magnitudes): their bit patterns order as
// unsigned integers, so each level is one v_max_u32 with a DPP operand.
__device__ __forceinline__ float tf_row16_max_nonneg(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = max(u, (uint32_t)tf_dppi<TF_DPP_QUAD_1032>((int)u));
    u = max(u, (uint32_t)tf_dppi<TF_DPP_QUAD_2301>((int)u));
    u = max(u, (uint32_t)tf_dppi<TF_DPP_ROW_HALF_MIRROR>((int)u));
    u = max(u, (uint32_t)tf_dppi<TF_DPP_ROW_MIRROR>((int)u));
    return __builtin_bit_cast(float, u);
}

// Maximum over aligned 32-lane groups; every lane receives it.
__device__ __forceinline__ float tf_group32_max(float v) {
    v = tf_row16_max(v);
    return fmaxf(v, tf_swap16(v));
}

// Maximum over the wave; every lane receives it.
__device__ __forceinline__ float tf_wave_max(float v) {
    v = tf_group32_max(v);
    return fmaxf(tf_readlane(v, 0), tf_readlane(v, 32));
}

// Global wave id of a persistent grid, numbered block-major: wave w of
// block b is w * gridDim.x + b, so consecutive tasks (task = id + k * total)
// go to different workgroups and every CU gets within one task of the same
// share.
__device__ __forceinline__ int tf_wave_id() {
    return (int)((threadIdx.x >> 6) * gridDim.x + blockIdx.x);
}

// ---------------------------------------------------------- vector loads

typedef uint32_t tf_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t tf_u32x2 __attribute__((ext_vector_type(2)));
// 16-byte / 8-byte loads from addresses that are only 4-byte aligned
// (212-byte Q6_K blocks).  gfx950 global_load_dwordx4 needs dword alignment.
struct __attribute__((packed, aligned(4))) tf_a4x4 { tf_u32x4 v; };
struct __attribute__((packed, aligned(4))) tf_a4x2 { tf_u32x2 v; };

// Global memory (address space 1).  The weight and cache loads below name
// it explicitly: a pointer the compiler cannot trace to a kernel argument
// (one read from a table in memory) would otherwise become a flat access,
// which also counts against the LDS wait counter and so makes every LDS
// wait drain the weight loads in flight.
#define TF_GAS __attribute__((address_space(1)))

__device__ __forceinline__ tf_u32x4 tf_ld16(const void* p) {
    return *(const TF_GAS tf_u32x4*)p;
}
__device__ __forceinline__ tf_u32x4 tf_ld16_a4(const void* p) {
    return ((const TF_GAS tf_a4x4*)p)->v;
}
__device__ __forceinline__ tf_u32x2 tf_ld8_a4(const void* p) {
    return ((const TF_GAS tf_a4x2*)p)->v;
}
// One value of type T (a scalar) from global memory.
template <class T>
__device__ __forceinline__ T tf_gld(const T* p) {
    return *(const TF_GAS T*)p;
}
// Two consecutive floats from global memory (8-byte aligned).
__device__ __forceinline__ float2 tf_gld2(const float* p) {
    const unsigned long long v = *(const TF_GAS unsigned long long*)p;
    return make_float2(__uint_as_float((unsigned)v), __uint_as_float((unsigned)(v >> 32)));
}

// ---------------------------------------------------------------- Q8 math

// One value of the Q8 activation format used by the reference
// (kernels/gemv.cu:36-37): q = amax == 0 ? 0 : rint_even(x / d) with
// d = amax * fl(1/127) and an IEEE-correct division.
//
// The division is avoided where it cannot matter: with r = v_rcp(d) (1 ulp)
// and |x / d| <= 127.x, y = x * r is within 2^-15 of RN(x / d), so when y's
// fraction lies farther than 2^-14 from 0.5 both round to the same integer.
// Otherwise (about 1e-4 of the values), or for a subnormal / zero d, the
// IEEE division decides.  The result is that of rint_even(RN(x / d)).
__device__ __forceinline__ int tf_q8_value_r(float x, float amax, float d, float r) {
    const float y = x * r;
    const float fr = fabsf(y - __builtin_truncf(y));
    const bool risky = !(d >= 1.17549435e-38f) || fabsf(fr - 0.5f) < 6.103515625e-05f;
    float q = y;
    if (risky) q = x / (amax == 0.f ? 1.f : d);
    return amax == 0.f ? 0 : (int)__builtin_rintf(q);
}

__device__ __forceinline__ int tf_q8_value(float x, float amax, float d) {
    return tf_q8_value_r(x, amax, d, __builtin_amdgcn_rcpf(d));
}

// Q8 of one 32-value group held as pairs: lane m (= lane & 15) of a
// 16-lane row holds values 2m and 2m+1.  Every reduction is a DPP row
// operation.  Returns the two q values and the group scale d; s_half is the
// int sum of q over this lane's 16-value half (lanes 0-7 / 8-15), s_other
// the other half's; f_half (when WITH_F32) the f32 sum of x over the half as
// the pairwise tree ((x0+x1)+(x2+x3)) + ((x4+x5)+(x6+x7)) + ... of pairs.
struct TfQ8Pair {
    int q0, q1;
    float d;
    int s_half, s_other;
    float f_half;
};

template <bool WITH_F32>
__device__ __forceinline__ TfQ8Pair tf_q8_pair(float x0, float x1) {
    TfQ8Pair r;
    const float amax = tf_row16_max_nonneg(fmaxf(fabsf(x0), fabsf(x1)));
    r.d = amax * (1.0f / 127.0f);
    const float rcp = __builtin_amdgcn_rcpf(r.d);
    r.q0 = tf_q8_value_r(x0, amax, r.d, rcp);
    r.q1 = tf_q8_value_r(x1, amax, r.d, rcp);
    int s = r.q0 + r.q1;
    s += tf_dppi<TF_DPP_QUAD_1032>(s);
    s += tf_dppi<TF_DPP_QUAD_2301>(s);
    s += tf_dppi<TF_DPP_ROW_HALF_MIRROR>(s);
    r.s_half = s;
    r.s_other = tf_dppi<TF_DPP_ROW_MIRROR>(s);
    r.f_half = 0.f;
    if (WITH_F32) {
        float f = x0 + x1;
        f += tf_dpp<TF_DPP_QUAD_1032>(f);
        f += tf_dpp<TF_DPP_QUAD_2301>(f);
        f += tf_dpp<TF_DPP_ROW_HALF_MIRROR>(f);
        r.f_half = f;
    }
    return r;
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
