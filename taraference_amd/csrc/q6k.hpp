// Q6_K building blocks shared by the Q6_K GEMV kernels.
//
// Q6_K super-block (256 values; kernels/common.cu:164-186):
//   ql[128] @0, qh[64] @128, int8 scales[16] @192, d (f16) @208.
//   For half n (0,1) and l in 0..31:
//     value 128n+l    = (ql[64n+l]    & 15) | ((qh[32n+l] >> 0) & 3) << 4
//     value 128n+32+l = (ql[64n+32+l] & 15) | ((qh[32n+l] >> 2) & 3) << 4
//     value 128n+64+l = (ql[64n+l]    >> 4) | ((qh[32n+l] >> 4) & 3) << 4
//     value 128n+96+l = (ql[64n+32+l] >> 4) | ((qh[32n+l] >> 6) & 3) << 4
//   weight = d * scales[v/16] * (value - 32).
// The reference repacks blocks to 212 bytes (cuda/load.rs:145-159) so that
// every block starts on a dword; the f32-activation path reads raw 210-byte
// blocks.
//
// Lane part p = lane & 3 of a 4-lane slot: n = p >> 1, h = p & 1.  It loads
// ql[64n+16h, +16), ql[64n+32+16h, +16) and qh[32n+16h, +16), which hold the
// 64 values 128n + 32k + 16h + i (k = 0..3, i = 0..15): four 16-value scale
// groups 8n + 2k + h, i.e. a quarter of the super-block.
#pragma once
#include "stage.hpp"

struct TfQ6kPart {
    tf_u32x4 a;   // ql[64n+16h ..]
    tf_u32x4 b;   // ql[64n+32+16h ..]
    tf_u32x4 hq;  // qh[32n+16h ..]
    tf_u32x2 sc;  // scales[8n .. 8n+8)
    uint32_t d;   // bytes 208..211 (d in the low half)
};

// 212-byte compact blocks: every field is dword aligned.
__device__ __forceinline__ void tf_q6k_load_c(const uint8_t* blk, int p, TfQ6kPart& q) {
    const int n = p >> 1, h = p & 1;
    q.a = tf_ld16_a4(blk + 64 * n + 16 * h);
    q.b = tf_ld16_a4(blk + 64 * n + 32 + 16 * h);
    q.hq = tf_ld16_a4(blk + 128 + 32 * n + 16 * h);
    q.sc = tf_ld8_a4(blk + 192 + 8 * n);
    q.d = tf_gld(reinterpret_cast<const uint32_t*>(blk + 208));
}

// 210-byte raw blocks: only 2-byte alignment is guaranteed.
__device__ __forceinline__ tf_u32x4 tf_ld16_a2(const uint8_t* p) {
    const TF_GAS uint16_t* s = (const TF_GAS uint16_t*)p;
    tf_u32x4 v;
    v.x = s[0] | ((uint32_t)s[1] << 16);
    v.y = s[2] | ((uint32_t)s[3] << 16);
    v.z = s[4] | ((uint32_t)s[5] << 16);
    v.w = s[6] | ((uint32_t)s[7] << 16);
    return v;
}
__device__ __forceinline__ void tf_q6k_load_r(const uint8_t* blk, int p, TfQ6kPart& q) {
    const int n = p >> 1, h = p & 1;
    q.a = tf_ld16_a2(blk + 64 * n + 16 * h);
    q.b = tf_ld16_a2(blk + 64 * n + 32 + 16 * h);
    q.hq = tf_ld16_a2(blk + 128 + 32 * n + 16 * h);
    const TF_GAS uint16_t* s2 = (const TF_GAS uint16_t*)(blk + 192 + 8 * n);
    q.sc = tf_u32x2{s2[0] | ((uint32_t)s2[1] << 16), s2[2] | ((uint32_t)s2[3] << 16)};
    q.d = ((const TF_GAS uint16_t*)(blk + 208))[0];
}

// Unsigned 6-bit values (0..63) of dword i of value group k, 4 per dword.
__device__ __forceinline__ uint32_t tf_q6k_word(const TfQ6kPart& q, int k, int i) {
    const uint32_t M = 0x0f0f0f0fu, H = 0x30303030u;
    const uint32_t a = q.a[i], b = q.b[i], hq = q.hq[i];
    switch (k) {
    case 0: return (a & M) | ((hq << 4) & H);
    case 1: return (b & M) | ((hq << 2) & H);
    case 2: return ((a >> 4) & M) | (hq & H);
    default: return ((b >> 4) & M) | ((hq >> 2) & H);
    }
}

// Signed scale of value group k for lane part p.
__device__ __forceinline__ int tf_q6k_scale(const TfQ6kPart& q, int p, int k) {
    const int h = p & 1;
    const uint32_t w = k < 2 ? q.sc.x : q.sc.y;  // scales 8n..8n+3 / 8n+4..8n+7
    const int shift = 8 * h + 16 * (k & 1);
    return (int)__builtin_amdgcn_sbfe(w, shift, 8);
}

// Exact integer stage: idot[k] = sum (q6 - 32) * q8 over scale group
// 8n + 2k + h.  q8sb points at the super-block's Q8 bytes in the padded LDS
// image (value byte o at q8sb + tf_q8_pad(o)) and
// s16 at its 16 per-16-value q8 sums.
__device__ __forceinline__ void tf_q6k_idots(const TfQ6kPart& q, int p, const int8_t* q8sb,
                                             const int32_t* s16, int idot[4]) {
    const int n = p >> 1, h = p & 1;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const tf_u32x4 u =
            *reinterpret_cast<const tf_u32x4*>(q8sb + tf_q8_pad(128 * n + 32 * k + 16 * h));
        int s = tf_dot4((int)tf_q6k_word(q, k, 0), (int)u.x, 0);
        s = tf_dot4((int)tf_q6k_word(q, k, 1), (int)u.y, s);
        s = tf_dot4((int)tf_q6k_word(q, k, 2), (int)u.z, s);
        s = tf_dot4((int)tf_q6k_word(q, k, 3), (int)u.w, s);
        idot[k] = s - 32 * s16[8 * n + 2 * k + h];
    }
}

// The activation image in LDS (q8, d8, s16 = per-16-value q8 sums) is built
// by tf_stage_act (stage.hpp).
using TfQ6Lds = TfAct;

// fp32 contribution of this lane's quarter of super-block sb.
__device__ __forceinline__ float tf_q6k_part_dot(const TfQ6kPart& q, int p, int sb,
                                                 const TfQ6Lds& x) {
    int idot[4];
    tf_q6k_idots(q, p, x.q8 + sb * 320, x.s16 + sb * 16, idot);
    const int n = p >> 1;
    const float d = tf_h2f(q.d);
    const float4 d8 = *reinterpret_cast<const float4*>(x.d8 + sb * 8 + 4 * n);
    float acc = (float)(tf_q6k_scale(q, p, 0) * idot[0]) * d8.x;
    acc += (float)(tf_q6k_scale(q, p, 1) * idot[1]) * d8.y;
    acc += (float)(tf_q6k_scale(q, p, 2) * idot[2]) * d8.z;
    acc += (float)(tf_q6k_scale(q, p, 3) * idot[3]) * d8.w;
    return d * acc;
}

template <int ITERS>
struct TfQ6kRow {
    TfQ6kPart q[ITERS];
};

template <int SPR, int ITERS>
__device__ __forceinline__ void tf_q6k_row_load(const uint8_t* __restrict__ col, bool valid,
                                                int sb0, int sb1, int sir, int p,
                                                TfQ6kRow<ITERS>& r) {
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int sb = sb0 + sir + i * SPR;
        if (valid && sb < sb1) tf_q6k_load_c(col + (size_t)sb * 212, p, r.q[i]);
    }
}

// The same loads issued unconditionally (a super-block past the row reloads
// super-block 0; tf_q6k_row_partial skips it), so the compiler can wait for
// exactly the loads a computation needs.
template <int SPR, int ITERS>
__device__ __forceinline__ void tf_q6k_row_load_u(const uint8_t* __restrict__ col, int nb, int sir,
                                                  int p, TfQ6kRow<ITERS>& r) {
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int sb = sir + i * SPR;
        tf_q6k_load_c(col + (size_t)(sb < nb ? sb : 0) * 212, p, r.q[i]);
    }
}

template <int SPR, int ITERS>
__device__ __forceinline__ float tf_q6k_row_partial(const TfQ6kRow<ITERS>& r, bool valid,
                                                    int sb0, int sb1, int sir, int p,
                                                    const TfQ6Lds& x) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int sb = sb0 + sir + i * SPR;
        if (valid && sb < sb1) acc += tf_q6k_part_dot(r.q[i], p, sb, x);
    }
    return acc;
}

template <int SPR>
__device__ __forceinline__ float tf_q6k_row_partial_loop(const uint8_t* __restrict__ col,
                                                         bool valid, int sb0, int sb1, int sir,
                                                         int p, const TfQ6Lds& x) {
    float acc = 0.f;
    for (int sb = sb0 + sir; valid && sb < sb1; sb += SPR) {
        TfQ6kPart q;
        tf_q6k_load_c(col + (size_t)sb * 212, p, q);
        acc += tf_q6k_part_dot(q, p, sb, x);
    }
    return acc;
}

// f32-activation contribution of this lane's quarter of a raw (210-byte)
// super-block sb (kernels/gemv.cu:233-264 arithmetic): per scale group,
// sum(q*x) - 32*sum(x), scaled by d*sc.  act.xf / act.xs16 hold the
// normalized activation and its 16-value sums.
__device__ __forceinline__ float tf_q6k_f32_part_dot(const TfQ6kPart& q, int p, int sb,
                                                     const TfAct& act) {
    const int n = p >> 1, h = p & 1;
    const float d = tf_h2f(q.d);
    float part = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float* xv = act.xf + sb * 256 + 128 * n + 32 * k + 16 * h;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t word = tf_q6k_word(q, k, i);
            const float4 xx = *reinterpret_cast<const float4*>(xv + 4 * i);
            s += (float)(word & 0xff) * xx.x;
            s += (float)((word >> 8) & 0xff) * xx.y;
            s += (float)((word >> 16) & 0xff) * xx.z;
            s += (float)(word >> 24) * xx.w;
        }
        s -= 32.f * act.xs16[sb * 16 + 8 * n + 2 * k + h];
        part += (float)tf_q6k_scale(q, p, k) * s;
    }
    return d * part;
}
