// Fused argmax over GEMV outputs (replaces argmax_f32, kernels/ops.cu:573-599,
// after the lm_head GEMV).  Each output j is turned into a 64-bit key
// (ordered float bits << 32 | ~j) whose unsigned maximum is the largest value
// with the lowest index among exact ties.  Waves max-merge their keys into
// TF_ARGMAX_SLOTS slots (wave w -> slot w % TF_ARGMAX_SLOTS): atomics to a
// single address serialize at the memory side across the XCDs, ~9 ns each,
// while 1024 distinct addresses spread them over the channels.
#pragma once
#include "tf_common.hpp"

__device__ __forceinline__ unsigned long long tf_argmax_key(float v, int j) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)j);
}

__device__ __forceinline__ int tf_argmax_key_index(unsigned long long k) {
    return k ? (int)(0xFFFFFFFFu - (uint32_t)k) : 0;
}

__device__ __forceinline__ unsigned long long tf_wave_max_u64(unsigned long long k) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)k, off, 64);
        const uint32_t hi = __shfl_xor((uint32_t)(k >> 32), off, 64);
        const unsigned long long o = ((unsigned long long)hi << 32) | lo;
        k = o > k ? o : k;
    }
    return k;
}

// Reduce the slots and clear them for the next launch.  Called by all
// threads of one 256-thread block; every thread returns the maximum key.
__device__ __forceinline__ unsigned long long tf_argmax_slots_take(unsigned long long* slots) {
    __shared__ unsigned long long part[4];
    unsigned long long k = 0;
    for (int i = threadIdx.x; i < TF_ARGMAX_SLOTS; i += 256) {
        const unsigned long long v = slots[i];
        k = v > k ? v : k;
        slots[i] = 0ull;
    }
    k = tf_wave_max_u64(k);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = k;
    __syncthreads();
    k = part[0];
    for (int w = 1; w < 4; w++) k = part[w] > k ? part[w] : k;
    return k;
}
