// Fused argmax over GEMV outputs (replaces argmax_f32, kernels/ops.cu:573-599,
// launched as one 256-thread block by layer.rs:2248-2255).
//
// The reference's result, restated: thread t scans i = t, t+256, ... with a
// strict `v > best` from best = -1e30, so it keeps the first index of its
// residue class holding the class maximum; NaN and values <= -1e30 never
// win, and a class with none keeps index 0.  The 256 slots then merge in a
// halving tree where the lower slot wins ties, so among slots tied at the
// maximum the one whose 8-bit reversed slot number is smallest wins (even
// before odd, then 0 mod 4 before 2 mod 4, ...).  Values compare as floats,
// so -0 ties with +0.
//
// Here each output j becomes a 64-bit key whose unsigned maximum is exactly
// that winner: ordered float bits (with -0 folded onto +0) in the high word,
// and in the low word the complement of (bitrev8(j mod 256) << 24 | j / 256),
// the tie priority.  Excluded values (NaN, <= -1e30) give key 0, and key 0
// decodes to index 0, the reference's answer when nothing beats -1e30.
// Waves max-merge their keys into TF_ARGMAX_SLOTS slots (wave w -> slot
// w % TF_ARGMAX_SLOTS): atomics to a single address serialize at the memory
// side across the XCDs, ~9 ns each, while 1024 distinct addresses spread
// them over the channels.
#pragma once
#include "tf_common.hpp"

__device__ __forceinline__ uint32_t tf_bitrev8(uint32_t r) {
    return __builtin_bitreverse32(r) >> 24;
}

__device__ __forceinline__ unsigned long long tf_argmax_key(float v, int j) {
    if (!(v > -1e30f)) return 0ull;  // NaN and <= -1e30 never win
    if (v == 0.0f) v = 0.0f;        // -0 ties with +0
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint32_t prio = (tf_bitrev8((uint32_t)j & 255u) << 24) | ((uint32_t)j >> 8);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - prio);
}

__device__ __forceinline__ int tf_argmax_key_index(unsigned long long k) {
    if (!k) return 0;
    const uint32_t prio = 0xFFFFFFFFu - (uint32_t)k;
    return (int)(((prio & 0xFFFFFFu) << 8) | tf_bitrev8(prio >> 24));
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
