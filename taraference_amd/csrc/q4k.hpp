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
#include "tf_common.hpp"

struct TfQ8Lds {
    const int8_t* q8;   // nb*256 bytes
    const float* d8;    // nb*8
    const float* ds;    // nb*8: d8[g] * sum(q8 in group g)
};

// LDS bytes needed to stage the Q8 activation of nb super-blocks.
__host__ __device__ constexpr int tf_q8_lds_bytes(int nb) { return nb * 256 + nb * 8 * 8; }

__device__ __forceinline__ TfQ8Lds tf_q8_lds_view(uint8_t* lds, int nb) {
    TfQ8Lds v;
    v.q8 = reinterpret_cast<const int8_t*>(lds);
    v.d8 = reinterpret_cast<const float*>(lds + nb * 256);
    v.ds = reinterpret_cast<const float*>(lds + nb * 256 + nb * 32);
    return v;
}

// Copy a pre-quantized activation (groups [0, nb*8)) into LDS and derive
// ds[g].  Cooperative over the whole workgroup; ends with a barrier.
__device__ __forceinline__ void tf_stage_q8(const int8_t* __restrict__ xq,
                                            const float* __restrict__ xd,
                                            int nb, uint8_t* lds,
                                            int32_t* sums_out = nullptr) {
    int8_t* q8s = reinterpret_cast<int8_t*>(lds);
    float* d8s = reinterpret_cast<float*>(lds + nb * 256);
    float* dss = reinterpret_cast<float*>(lds + nb * 256 + nb * 32);
    const int groups = nb * 8;
    const bool a16 = ((uintptr_t)xq & 15) == 0;
    // one 32-byte group per thread: copy and sum in one pass
    for (int g = threadIdx.x; g < groups; g += blockDim.x) {
        tf_u32x4 a, b;
        if (a16) {
            a = tf_ld16(xq + g * 32);
            b = tf_ld16(xq + g * 32 + 16);
        } else {
            uint32_t w[8];
            for (int i = 0; i < 8; i++) {
                const uint8_t* p = reinterpret_cast<const uint8_t*>(xq) + g * 32 + 4 * i;
                w[i] = p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
            }
            a = tf_u32x4{w[0], w[1], w[2], w[3]};
            b = tf_u32x4{w[4], w[5], w[6], w[7]};
        }
        reinterpret_cast<tf_u32x4*>(q8s + g * 32)[0] = a;
        reinterpret_cast<tf_u32x4*>(q8s + g * 32)[1] = b;
        const int one = 0x01010101;
        int s = tf_dot4(one, (int)a.x, 0);
        s = tf_dot4(one, (int)a.y, s);
        s = tf_dot4(one, (int)a.z, s);
        s = tf_dot4(one, (int)a.w, s);
        s = tf_dot4(one, (int)b.x, s);
        s = tf_dot4(one, (int)b.y, s);
        s = tf_dot4(one, (int)b.z, s);
        s = tf_dot4(one, (int)b.w, s);
        const float d = xd[g];
        d8s[g] = d;
        dss[g] = d * (float)s;
        if (sums_out) sums_out[g] = s;
    }
    __syncthreads();
}

// Quantize an f32 activation (nb*256 values) straight into LDS, bit-identical
// to tf_quantize_q8 (kernels/gemv.cu:16-40 quantize_q8_smem).  Each wave
// quantizes two 32-value groups per step (lanes 0-31 / 32-63); the loads of
// eight steps are issued before any of them is used.  Ends with a barrier.
__device__ __forceinline__ void tf_quantize_to_lds(const float* __restrict__ x,
                                                   int nb, uint8_t* lds) {
    int8_t* q8s = reinterpret_cast<int8_t*>(lds);
    float* d8s = reinterpret_cast<float*>(lds + nb * 256);
    float* dss = reinterpret_cast<float*>(lds + nb * 256 + nb * 32);
    const int groups = nb * 8;
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31;
    const int waves = blockDim.x >> 6;
    const int gstep = 2 * waves;
    const int g0 = (threadIdx.x >> 6) * 2 + (lane >> 5);
    const int iters = (groups + gstep - 1) / gstep;
    for (int i0 = 0; i0 < iters; i0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int g = g0 + gstep * (i0 + u);
            v[u] = (i0 + u < iters && g < groups) ? x[g * 32 + l32] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (i0 + u < iters) {  // wave-uniform
                const int g = g0 + gstep * (i0 + u);
                const float xi = v[u];
                const float amax = tf_group32_max(fabsf(xi));
                const float d = amax * (1.0f / 127.0f);
                const int q = tf_q8_value(xi, amax, d);
                int s = q;
                s += __shfl_xor(s, 1, 64);
                s += __shfl_xor(s, 2, 64);
                s += __shfl_xor(s, 4, 64);
                s += __shfl_xor(s, 8, 64);
                s += __shfl_xor(s, 16, 64);
                if (g < groups) {
                    q8s[g * 32 + l32] = (int8_t)q;
                    if (l32 == 0) {
                        d8s[g] = d;
                        dss[g] = d * (float)s;
                    }
                }
            }
        }
    }
    __syncthreads();
}

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

// Exact integer stage: dlo = sum q4*q8 over sub-block 2t, dhi over 2t+1.
// q8g points at the 64 LDS bytes of groups 2t, 2t+1 of this super-block.
__device__ __forceinline__ void tf_q4k_idots(const TfQ4kPart& p, const int8_t* q8g,
                                             int& dlo, int& dhi) {
    const tf_u32x4* qv = reinterpret_cast<const tf_u32x4*>(q8g);
    const tf_u32x4 u0 = qv[0], u1 = qv[1], w0 = qv[2], w1 = qv[3];
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

// fp32 contribution of this lane's two sub-blocks of super-block sb.
__device__ __forceinline__ float tf_q4k_part_dot(const TfQ4kPart& p, int t, int sb,
                                                 const TfQ8Lds& x) {
    int dlo, dhi;
    tf_q4k_idots(p, x.q8 + sb * 256 + 64 * t, dlo, dhi);
    int sc0, sc1, m0, m1;
    tf_q4k_scales(p.h, t, sc0, sc1, m0, m1);
    const float d = tf_h2f(p.h.x);
    const float dmin = tf_h2f(p.h.x >> 16);
    const int g = sb * 8 + 2 * t;
    const float2 d8 = *reinterpret_cast<const float2*>(x.d8 + g);
    const float2 ds = *reinterpret_cast<const float2*>(x.ds + g);
    const float scale_term = d8.x * (float)(dlo * sc0) + d8.y * (float)(dhi * sc1);
    const float min_term = (float)m0 * ds.x + (float)m1 * ds.y;
    return d * scale_term - dmin * min_term;
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
