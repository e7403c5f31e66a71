// Activation staging for the GEMV kernels: every workgroup builds, in LDS,
// the image of the activation its rows consume, from one of three sources:
//   TF_SRC_Q8   pre-quantized Q8 (q8 bytes + d8) in global memory;
//   TF_SRC_F32  an f32 vector, quantized here (kernels/gemv.cu:16-40);
//   TF_SRC_NORM an f32 vector that is first RMS-normalized and scaled by a
//               weight (kernels/ops.cu:4-34, same summation order), then
//               quantized.
// Quantization is bit-identical to tf_quantize_q8 (IEEE division,
// round-half-even), so a fused prologue produces the same Q8 bytes as the
// separate kernels would.
//
// LDS image for nb super-blocks (G = 8*nb groups of 32 values):
//   q8[256*nb] int8 | d8[G] f32 | ds[G] f32 = d8*sum32(q8) |
//   s16[2G] i32 = per-16 sums of q8 | (optional) xf[256*nb] f32 normalized
//   activation | xs16[2G] f32 = per-16 sums of xf
// The Q4_K x Q8 path reads q8/d8/ds, the Q6_K x Q8 path q8/d8/s16 and the
// Q6_K x f32 path xf/xs16.
#pragma once
#include "tf_common.hpp"

enum TfSrc { TF_SRC_Q8 = 0, TF_SRC_F32 = 1, TF_SRC_NORM = 2 };

struct TfAct {
    const int8_t* q8;
    const float* d8;
    const float* ds;
    const int32_t* s16;
    const float* xf;
    const float* xs16;
};

__host__ __device__ constexpr int tf_act_lds_bytes(int nb, bool with_f32) {
    return nb * 256 + nb * 8 * 4 * 2 + nb * 16 * 4 + (with_f32 ? nb * 256 * 4 + nb * 16 * 4 : 0);
}

__device__ __forceinline__ TfAct tf_act_view(uint8_t* lds, int nb) {
    TfAct a;
    a.q8 = reinterpret_cast<const int8_t*>(lds);
    a.d8 = reinterpret_cast<const float*>(lds + nb * 256);
    a.ds = a.d8 + nb * 8;
    a.s16 = reinterpret_cast<const int32_t*>(a.ds + nb * 8);
    a.xf = reinterpret_cast<const float*>(a.s16 + nb * 16);
    a.xs16 = a.xf + nb * 256;
    return a;
}

struct TfActSrc {
    int kind;             // TfSrc
    const int8_t* xq;     // TF_SRC_Q8
    const float* xd;      // TF_SRC_Q8
    const float* x;       // TF_SRC_F32 / TF_SRC_NORM; with TF_SRC_Q8 the f32
                          // vector behind the Q8 bytes (copied when WITH_F32)
    const float* norm_w;  // TF_SRC_NORM
    float eps;            // TF_SRC_NORM
};

// Reference-order RMS scale over n = 256*nb values with a 256-thread block:
// strided per-thread sums, halving tree (kernels/ops.cu:17-29).
__device__ __forceinline__ float tf_rms_scale_256(const float* __restrict__ x, int n, float eps,
                                                  float* red /* 256 floats of LDS */) {
    float local = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = x[i];
        local = fmaf(v, v, local);  // fused, as under fmad=true
    }
    red[threadIdx.x] = local;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    const float scale = 1.0f / sqrtf(red[0] / (float)n + eps);
    __syncthreads();
    return scale;
}

// Build the LDS image.  Must be called by all 256 threads; ends with a
// barrier.  WITH_F32 also keeps the (normalized) f32 activation.
template <bool WITH_F32>
__device__ __forceinline__ void tf_stage_act(const TfActSrc& src, int nb, uint8_t* lds) {
    int8_t* q8s = reinterpret_cast<int8_t*>(lds);
    float* d8s = reinterpret_cast<float*>(lds + nb * 256);
    float* dss = d8s + nb * 8;
    int32_t* s16 = reinterpret_cast<int32_t*>(dss + nb * 8);
    float* xf = reinterpret_cast<float*>(s16 + nb * 16);
    float* xs16 = xf + nb * 256;
    const int groups = nb * 8;
    if (src.kind == TF_SRC_Q8) {
        const bool a16 = ((uintptr_t)src.xq & 15) == 0;
        for (int g = threadIdx.x; g < groups; g += blockDim.x) {
            tf_u32x4 a, b;
            if (a16) {
                a = tf_ld16(src.xq + g * 32);
                b = tf_ld16(src.xq + g * 32 + 16);
            } else {
                uint32_t w[8];
                for (int i = 0; i < 8; i++) {
                    const uint8_t* p = reinterpret_cast<const uint8_t*>(src.xq) + g * 32 + 4 * i;
                    w[i] = p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
                }
                a = tf_u32x4{w[0], w[1], w[2], w[3]};
                b = tf_u32x4{w[4], w[5], w[6], w[7]};
            }
            reinterpret_cast<tf_u32x4*>(q8s + g * 32)[0] = a;
            reinterpret_cast<tf_u32x4*>(q8s + g * 32)[1] = b;
            const int one = 0x01010101;
            int sa = tf_dot4(one, (int)a.x, 0);
            sa = tf_dot4(one, (int)a.y, sa);
            sa = tf_dot4(one, (int)a.z, sa);
            sa = tf_dot4(one, (int)a.w, sa);
            int sb = tf_dot4(one, (int)b.x, 0);
            sb = tf_dot4(one, (int)b.y, sb);
            sb = tf_dot4(one, (int)b.z, sb);
            sb = tf_dot4(one, (int)b.w, sb);
            const float d = src.xd[g];
            d8s[g] = d;
            dss[g] = d * (float)(sa + sb);
            s16[2 * g] = sa;
            s16[2 * g + 1] = sb;
        }
        if (WITH_F32 && src.x) {
            // one 16-value run per thread: copy, and sum as the pairwise tree
            // that the xor butterfly of the f32 sources forms (bit-identical)
            for (int i = threadIdx.x; i < nb * 16; i += blockDim.x) {
                float t[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float4 v = *reinterpret_cast<const float4*>(src.x + i * 16 + 4 * k);
                    *reinterpret_cast<float4*>(xf + i * 16 + 4 * k) = v;
                    t[k] = (v.x + v.y) + (v.z + v.w);
                }
                xs16[i] = (t[0] + t[1]) + (t[2] + t[3]);
            }
        }
        __syncthreads();
        return;
    }
    __shared__ float red[256];
    float scale = 1.f;
    if (src.kind == TF_SRC_NORM) scale = tf_rms_scale_256(src.x, nb * 256, src.eps, red);
    // lanes 0-31 / 32-63 of a wave quantize one group each per step; the
    // loads of eight steps are issued before they are used.
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
            float xv = 0.f;
            if (i0 + u < iters && g < groups) {
                xv = src.x[g * 32 + l32];
                if (src.kind == TF_SRC_NORM) xv = xv * scale * src.norm_w[g * 32 + l32];
            }
            v[u] = xv;
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
                s += __shfl_xor(s, 8, 64);  // sum over the 16-lane half
                const int s_other = __shfl_xor(s, 16, 64);
                float fs = 0.f;
                if (WITH_F32) {
                    fs = xi;
                    fs += __shfl_xor(fs, 1, 64);
                    fs += __shfl_xor(fs, 2, 64);
                    fs += __shfl_xor(fs, 4, 64);
                    fs += __shfl_xor(fs, 8, 64);
                }
                if (g < groups) {
                    q8s[g * 32 + l32] = (int8_t)q;
                    if (WITH_F32) xf[g * 32 + l32] = xi;
                    if ((l32 & 15) == 0) {
                        s16[2 * g + (l32 >> 4)] = s;
                        if (WITH_F32) xs16[2 * g + (l32 >> 4)] = fs;
                    }
                    if (l32 == 0) {
                        d8s[g] = d;
                        dss[g] = d * (float)(s + s_other);
                    }
                }
            }
        }
    }
    __syncthreads();
}
