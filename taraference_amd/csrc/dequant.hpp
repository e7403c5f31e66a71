// Single-value dequantization of Q4_K and Q6_K super-blocks, used where a
// whole row is expanded to f32 (the token embedding).
#pragma once
#include "tf_common.hpp"

// One 256-value super-block per wave-quarter: value v of block bi.
// Q4_K: d*sc*q - dmin*m (kernels/common.cu:64-84); Q6_K: d*sc*(q-32)
// (kernels/common.cu:164-186).  Both products are exact in fp32, so the row
// is bit-identical to any evaluation order.
__device__ __forceinline__ float tf_q4k_value(const uint8_t* blk_, int v) {
    const TF_GAS uint8_t* blk = (const TF_GAS uint8_t*)blk_;
    const float d = tf_h2f(blk[0] | (blk[1] << 8));
    const float dmin = tf_h2f(blk[2] | (blk[3] << 8));
    const TF_GAS uint8_t* sc = blk + 4;
    const int g = v >> 5, t = v >> 6, l = v & 31;
    int s, m;
    if (g < 4) {
        s = sc[g] & 63;
        m = sc[g + 4] & 63;
    } else {
        s = (sc[g + 4] & 0xF) | ((sc[g - 4] >> 6) << 4);
        m = (sc[g + 4] >> 4) | ((sc[g] >> 6) << 4);
    }
    const uint8_t qb = blk[16 + 32 * t + l];
    const int q = (g & 1) ? (qb >> 4) : (qb & 0xF);
    const float d1 = d * (float)s, m1 = dmin * (float)m;
    return d1 * (float)q - m1;
}

__device__ __forceinline__ float tf_q6k_value(const uint8_t* blk_, int v) {
    const TF_GAS uint8_t* blk = (const TF_GAS uint8_t*)blk_;
    const int n = v >> 7, r = v & 127, k = r >> 5, l = r & 31;
    const TF_GAS uint8_t* ql = blk + 64 * n;
    const uint8_t qh = blk[128 + 32 * n + l];
    int lo;
    switch (k) {
    case 0: lo = ql[l] & 0xF; break;
    case 1: lo = ql[32 + l] & 0xF; break;
    case 2: lo = ql[l] >> 4; break;
    default: lo = ql[32 + l] >> 4; break;
    }
    const int q = (lo | (((qh >> (2 * k)) & 3) << 4)) - 32;
    const float d = tf_h2f(blk[208] | (blk[209] << 8));
    const int8_t sc = (int8_t)blk[192 + (v >> 4)];
    return d * (float)sc * (float)q;
}

// Q8_0 (34-byte blocks of 32): d * qs[v]; Q5_0 (22-byte blocks of 32):
// d * (code - 16) (kernels/embed.cu embed_q8_0 / embed_q5_0).  Value v of
// the block at blk.
__device__ __forceinline__ float tf_q8_0_value(const uint8_t* blk_, int v) {
    const TF_GAS uint8_t* blk = (const TF_GAS uint8_t*)blk_;
    return tf_h2f(blk[0] | (blk[1] << 8)) * (float)(int8_t)blk[2 + v];
}

__device__ __forceinline__ float tf_q5_0_value(const uint8_t* blk_, int v) {
    const TF_GAS uint8_t* blk = (const TF_GAS uint8_t*)blk_;
    const uint32_t qh = blk[2] | (blk[3] << 8) | (blk[4] << 16) | ((uint32_t)blk[5] << 24);
    const int t = v & 15;
    const int nib = v < 16 ? (blk[6 + t] & 0xF) : (blk[6 + t] >> 4);
    const int code = nib | (int)(((qh >> v) & 1u) << 4);
    return tf_h2f(blk[0] | (blk[1] << 8)) * (float)(code - 16);
}

// Value i of a row stored in blocks of block_bytes (144 / 210: 256 values,
// 34 / 22: 32 values).
template <int BB>
__device__ __forceinline__ float tf_row_value(const uint8_t* row, int i) {
    if constexpr (BB == 144) return tf_q4k_value(row + (size_t)(i >> 8) * 144, i & 255);
    else if constexpr (BB == 210) return tf_q6k_value(row + (size_t)(i >> 8) * 210, i & 255);
    else if constexpr (BB == 34) return tf_q8_0_value(row + (size_t)(i >> 5) * 34, i & 31);
    else return tf_q5_0_value(row + (size_t)(i >> 5) * 22, i & 31);
}
