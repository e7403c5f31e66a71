// Q4_K x Q8 building blocks shared by every Q4_K GEMV kernel.
//
// Q4_K super-block (144 B, 256 values; kernels/common.cu:40-84):
//   bytes 0..1 d (f16), 2..3 dmin (f16), 4..15 packed 6-bit scales/mins,
//   16..143 qs: qs[32t+l] low nibble = value 64t+l (sub-block 2t),
//               high nibble = value 64t+32+l (sub-block 2t+1).
//   value = d*sc[g]*q - dmin*m[g].
//
// Work split on gfx950: a "slot" of four consecutive lanes owns one
// super-block.  Lane part t = lane & 3 loads the 16-byte header and the 32
// qs bytes [32t, 32t+32) with three global_load_dwordx4, i.e. sub-blocks 2t
// and 2t+1 entirely.  A wave has 16 slots.  A row of nb super-blocks is
// spread over SPR slots (SPR = 4, 8 or 16), so one wave pass covers
// 16/SPR rows ("units"), each unit being 4*SPR contiguous lanes.
//
// The Q8 activation lives in LDS: q8 bytes, d8[g], and ds[g] = d8[g]*sum(q8
// over group g), the latter turning the dmin term into two FMAs per lane.
#pragma once
#include "stage.hpp"

// The activation image in LDS (q8, d8, ds) is built by tf_stage_act
// (stage.hpp).
using TfQ8Lds = TfAct;

struct TfQ4kPart {
    tf_u32x4 h;  // d, dmin, scales[12]
    tf_u32x4 a;  // qs[32t .. 32t+16)
    tf_u32x4 b;  // qs[32t+16 .. 32t+32)
};

__device__ __forceinline__ void tf_q4k_load(const uint8_t* blk, int t, TfQ4kPart& p) {
    p.h = tf_ld16(blk);
    p.a = tf_ld16(blk + 16 + 32 * t);
    p.b = tf_ld16(blk + 32 + 32 * t);
}

// 6-bit scales and mins of sub-blocks 2t and 2t+1 (kernels/common.cu:40-50,
// in the 16-bit-pair form of kernels/gemv.cu:94-107).
__device__ __forceinline__ void tf_q4k_scales(const tf_u32x4& h, int t, int& sc0,
                                              int& sc1, int& m0, int& m1) {
    const uint32_t sh = (uint32_t)(t & 1) * 16u;
    const uint32_t a = h.y >> sh, b = h.z >> sh, c = h.w >> sh;
    const uint32_t sc_lo = a & 0x3f3fu, m_lo = b & 0x3f3fu;
    const uint32_t sc_hi = (c & 0x0f0fu) | ((a >> 2) & 0x3030u);
    const uint32_t m_hi = ((c >> 4) & 0x0f0fu) | ((b >> 2) & 0x3030u);
    const uint32_t scp = t < 2 ? sc_lo : sc_hi;
    const uint32_t mp = t < 2 ? m_lo : m_hi;
    sc0 = scp & 0xff;
    sc1 = (scp >> 8) & 0xff;
    m0 = mp & 0xff;
    m1 = (mp >> 8) & 0xff;
}

// Exact integer stage: dlo = sum q4*q8 over sub-block 2t, dhi over 2t+1,
// against the 64 Q8 bytes of groups 2t, 2t+1 (u0, u1: group 2t; w0, w1:
// group 2t + 1).
__device__ __forceinline__ void tf_q4k_idots_r(const TfQ4kPart& p, const tf_u32x4& u0,
                                               const tf_u32x4& u1, const tf_u32x4& w0,
                                               const tf_u32x4& w1, int& dlo, int& dhi) {
    const uint32_t M = 0x0f0f0f0fu;
    int lo = tf_dot4((int)(p.a.x & M), (int)u0.x, 0);
    lo = tf_dot4((int)(p.a.y & M), (int)u0.y, lo);
    lo = tf_dot4((int)(p.a.z & M), (int)u0.z, lo);
    lo = tf_dot4((int)(p.a.w & M), (int)u0.w, lo);
    lo = tf_dot4((int)(p.b.x & M), (int)u1.x, lo);
    lo = tf_dot4((int)(p.b.y & M), (int)u1.y, lo);
    lo = tf_dot4((int)(p.b.z & M), (int)u1.z, lo);
    lo = tf_dot4((int)(p.b.w & M), (int)u1.w, lo);
    int hi = tf_dot4((int)((p.a.x >> 4) & M), (int)w0.x, 0);
    hi = tf_dot4((int)((p.a.y >> 4) & M), (int)w0.y, hi);
    hi = tf_dot4((int)((p.a.z >> 4) & M), (int)w0.z, hi);
    hi = tf_dot4((int)((p.a.w >> 4) & M), (int)w0.w, hi);
    hi = tf_dot4((int)((p.b.x >> 4) & M), (int)w1.x, hi);
    hi = tf_dot4((int)((p.b.y >> 4) & M), (int)w1.y, hi);
    hi = tf_dot4((int)((p.b.z >> 4) & M), (int)w1.z, hi);
    hi = tf_dot4((int)((p.b.w >> 4) & M), (int)w1.w, hi);
    dlo = lo;
    dhi = hi;
}

// The same reading the bytes from LDS: q8g points at the 64 bytes of groups
// 2t, 2t+1 of this super-block (contiguous in the padded image too: the run
// is 64-byte aligned).
__device__ __forceinline__ void tf_q4k_idots(const TfQ4kPart& p, const int8_t* q8g,
                                             int& dlo, int& dhi) {
    const tf_u32x4* qv = reinterpret_cast<const tf_u32x4*>(q8g);
    tf_q4k_idots_r(p, qv[0], qv[1], qv[2], qv[3], dlo, dhi);
}

// The fp32 contribution from the exact integer sums dlo, dhi, the two
// groups' Q8 scales d8 and their d8 * sum(q8) ds.
__device__ __forceinline__ float tf_q4k_part_fp(const TfQ4kPart& p, int t, int dlo, int dhi,
                                                float2 d8, float2 ds) {
    int sc0, sc1, m0, m1;
    tf_q4k_scales(p.h, t, sc0, sc1, m0, m1);
    const float d = tf_h2f(p.h.x);
    const float dmin = tf_h2f(p.h.x >> 16);
    const float scale_term = d8.x * (float)(dlo * sc0) + d8.y * (float)(dhi * sc1);
    const float min_term = (float)m0 * ds.x + (float)m1 * ds.y;
    return d * scale_term - dmin * min_term;
}

// fp32 contribution of this lane's two sub-blocks of super-block sb.
__device__ __forceinline__ float tf_q4k_part_dot(const TfQ4kPart& p, int t, int sb,
                                                 const TfQ8Lds& x) {
    int dlo, dhi;
    tf_q4k_idots(p, x.q8 + tf_q8_pad(sb * 256 + 64 * t), dlo, dhi);
    const int g = sb * 8 + 2 * t;
    return tf_q4k_part_fp(p, t, dlo, dhi, *reinterpret_cast<const float2*>(x.d8 + g),
                          *reinterpret_cast<const float2*>(x.ds + g));
}

// The same reading the Q8 activation from global memory (xq 16-byte
// aligned): the 64 bytes of groups 2t, 2t+1, their scales, and the group
// sums formed here as the staging forms them (ds = d8 * (float)sum).
__device__ __forceinline__ float tf_q4k_part_dot_g(const TfQ4kPart& p, int t, int sb,
                                                   const int8_t* __restrict__ xq,
                                                   const float* __restrict__ xd) {
    const int8_t* q = xq + sb * 256 + 64 * t;
    const tf_u32x4 u0 = tf_ld16(q), u1 = tf_ld16(q + 16), w0 = tf_ld16(q + 32),
                   w1 = tf_ld16(q + 48);
    const int g = sb * 8 + 2 * t;
    const float2 d8 = *reinterpret_cast<const float2*>(xd + g);
    int dlo, dhi;
    tf_q4k_idots_r(p, u0, u1, w0, w1, dlo, dhi);
    const int one = 0x01010101;
    int s0 = tf_dot4(one, (int)u0.x, 0);
    s0 = tf_dot4(one, (int)u0.y, s0);
    s0 = tf_dot4(one, (int)u0.z, s0);
    s0 = tf_dot4(one, (int)u0.w, s0);
    s0 = tf_dot4(one, (int)u1.x, s0);
    s0 = tf_dot4(one, (int)u1.y, s0);
    s0 = tf_dot4(one, (int)u1.z, s0);
    s0 = tf_dot4(one, (int)u1.w, s0);
    int s1 = tf_dot4(one, (int)w0.x, 0);
    s1 = tf_dot4(one, (int)w0.y, s1);
    s1 = tf_dot4(one, (int)w0.z, s1);
    s1 = tf_dot4(one, (int)w0.w, s1);
    s1 = tf_dot4(one, (int)w1.x, s1);
    s1 = tf_dot4(one, (int)w1.y, s1);
    s1 = tf_dot4(one, (int)w1.z, s1);
    s1 = tf_dot4(one, (int)w1.w, s1);
    return tf_q4k_part_fp(p, t, dlo, dhi, d8, make_float2(d8.x * (float)s0, d8.y * (float)s1));
}

// Row dot split into a load phase and a compute phase so that kernels can
// keep the next task's weights in flight while computing the current one.
// A unit's lanes cover super-blocks sb0+sir, sb0+sir+SPR, ... < sb1; ITERS
// is ceil(max range / SPR) and bounds the unrolled register set.
template <int ITERS>
struct TfQ4kRow {
    TfQ4kPart p[ITERS];
};

template <int SPR, int ITERS>
__device__ __forceinline__ void tf_q4k_row_load(const uint8_t* __restrict__ col, bool valid,
                                                int sb0, int sb1, int sir, int t,
                                                TfQ4kRow<ITERS>& r) {
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int sb = sb0 + sir + i * SPR;
        if (valid && sb < sb1) tf_q4k_load(col + (size_t)sb * 144, t, r.p[i]);
    }
}

// The same loads issued unconditionally (a super-block past the row reloads
// super-block 0; tf_q4k_row_partial skips it): no branch around the loads,
// so the compiler can wait for exactly the loads a computation needs.
template <int SPR, int ITERS>
__device__ __forceinline__ void tf_q4k_row_load_u(const uint8_t* __restrict__ col, int nb,
                                                  int sir, int t, TfQ4kRow<ITERS>& r) {
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int sb = sir + i * SPR;
        tf_q4k_load(col + (size_t)(sb < nb ? sb : 0) * 144, t, r.p[i]);
    }
}

// Sum of this lane's parts; reduce with tf_group_sum<4*SPR> afterwards (all
// lanes of the wave must take part in that reduction).
template <int SPR, int ITERS>
__device__ __forceinline__ float tf_q4k_row_partial(const TfQ4kRow<ITERS>& r, bool valid,
                                                    int sb0, int sb1, int sir, int t,
                                                    const TfQ8Lds& x) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int sb = sb0 + sir + i * SPR;
        if (valid && sb < sb1) acc += tf_q4k_part_dot(r.p[i], t, sb, x);
    }
    return acc;
}

template <int SPR, int ITERS>
__device__ __forceinline__ float tf_q4k_row_partial_g(const TfQ4kRow<ITERS>& r, bool valid,
                                                      int nb, int sir, int t,
                                                      const int8_t* __restrict__ xq,
                                                      const float* __restrict__ xd) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int sb = sir + i * SPR;
        if (valid && sb < nb) acc += tf_q4k_part_dot_g(r.p[i], t, sb, xq, xd);
    }
    return acc;
}

// Runtime-length fallback for rows longer than the unrolled register set.
template <int SPR>
__device__ __forceinline__ float tf_q4k_row_partial_loop(const uint8_t* __restrict__ col,
                                                         bool valid, int sb0, int sb1, int sir,
                                                         int t, const TfQ8Lds& x) {
    float acc = 0.f;
    for (int sb = sb0 + sir; valid && sb < sb1; sb += SPR) {
        TfQ4kPart p;
        tf_q4k_load(col + (size_t)sb * 144, t, p);
        acc += tf_q4k_part_dot(p, t, sb, x);
    }
    return acc;
}
