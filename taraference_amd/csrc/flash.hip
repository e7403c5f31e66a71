// Split-KV flash decode for gfx950 (one query token).
//
// Replaces kernels/attn/flash.cu attn_flash_partial (:16), attn_flash_partial_d
// (:119) and attn_flash_reduce (:222).  The partial buffer keeps the
// reference layout partial[(h*n_split + s)*(2+hd)] = (m, l, O[hd]).
//
// A workgroup serves one (kv head, split) pair and every GQA query head that
// reads that kv head, so each K/V byte of the split is read once.  Its four
// waves walk the split in 64-token steps (wave w takes steps w, w+4, ...):
//   scores: lane = token; the lane streams its K row (16-byte loads) and
//           accumulates q_g . k for all G heads (q is wave-uniform);
//   softmax: per-head wave max / sum, online rescale (running m, l);
//   PV:     lane = head_dim/64 contiguous dims; every token's V row is one
//           coalesced 2*hd-byte load; exp weights are broadcast from LDS.
// The four per-wave states are merged with log-sum-exp in LDS at the end.
#include <math.h>

#include "tf_common.hpp"
#include "tf_host.hpp"

#define TF_FLASH_STEP 64
#define TF_FLASH_WAVES 4
#define TF_NEG_BIG (-1e30f)

template <int HD, int GMAX>
__global__ __launch_bounds__(256) void tf_flash_partial_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, float* __restrict__ partial, int n_head, int n_kv,
    int pos0, const int* __restrict__ pos0_dev, int n_split, float scale) {
    constexpr int DPL = HD / 64;  // dims per lane in the PV phase
    const int kv_h = blockIdx.x;
    const int s = blockIdx.y;
    const int G = n_head / n_kv;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int stride = n_kv * HD;
    if (pos0_dev) pos0 = pos0_dev[0];
    const int seq_len = pos0 + 1;
    const int chunk = (seq_len + n_split - 1) / n_split;
    const int t_begin = s * chunk;
    const int t_end = min(t_begin + chunk, seq_len);

    __shared__ float e_lds[TF_FLASH_WAVES][GMAX][TF_FLASH_STEP];
    __shared__ float m_lds[TF_FLASH_WAVES][GMAX];
    __shared__ float l_lds[TF_FLASH_WAVES][GMAX];
    __shared__ float o_lds[TF_FLASH_WAVES][GMAX][HD];

    const float* qk = q + (size_t)kv_h * G * HD;  // heads kv_h*G .. kv_h*G+G-1

    float m[GMAX], l[GMAX], o[GMAX][DPL];
#pragma unroll
    for (int g = 0; g < GMAX; g++) {
        m[g] = TF_NEG_BIG;
        l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; i++) o[g][i] = 0.f;
    }

    for (int t0 = t_begin + wave * TF_FLASH_STEP; t0 < t_end;
         t0 += TF_FLASH_WAVES * TF_FLASH_STEP) {
        // ---- scores (lane = token)
        const int t = t0 + lane;
        const bool tv = t < t_end;
        float sc[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; g++) sc[g] = 0.f;
        const uint16_t* krow = k_cache + (size_t)(tv ? t : t0) * stride + (size_t)kv_h * HD;
#pragma unroll 2
        for (int d = 0; d < HD; d += 8) {
            const tf_u32x4 kw = tf_ld16(krow + d);
            float kf[8];
            kf[0] = tf_h2f(kw.x);
            kf[1] = tf_h2f(kw.x >> 16);
            kf[2] = tf_h2f(kw.y);
            kf[3] = tf_h2f(kw.y >> 16);
            kf[4] = tf_h2f(kw.z);
            kf[5] = tf_h2f(kw.z >> 16);
            kf[6] = tf_h2f(kw.w);
            kf[7] = tf_h2f(kw.w >> 16);
#pragma unroll
            for (int g = 0; g < GMAX; g++) {
                if (g < G) {
                    const float* qg = qk + g * HD + d;
                    float a = sc[g];
#pragma unroll
                    for (int i = 0; i < 8; i++) a += qg[i] * kf[i];
                    sc[g] = a;
                }
            }
        }
        // ---- online softmax per head
        float alpha[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; g++) {
            if (g < G) {
                const float sv = tv ? sc[g] * scale : TF_NEG_BIG;
                float mx = sv;
                mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float m_new = fmaxf(m[g], mx);
                alpha[g] = __expf(m[g] - m_new);
                const float e = tv ? __expf(sv - m_new) : 0.f;
                e_lds[wave][g][lane] = e;
                const float tile_l = tf_group_sum<64>(e);
                l[g] = l[g] * alpha[g] + tile_l;
                m[g] = m_new;
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // ---- PV (lane = DPL dims)
#pragma unroll
        for (int g = 0; g < GMAX; g++)
#pragma unroll
            for (int i = 0; i < DPL; i++) o[g][i] *= (g < G) ? alpha[g] : 1.f;
        const int tlen = min(TF_FLASH_STEP, t_end - t0);
        const uint16_t* vbase = v_cache + (size_t)t0 * stride + (size_t)kv_h * HD + lane * DPL;
        for (int tt = 0; tt < tlen; tt++) {
            const uint16_t* vr = vbase + (size_t)tt * stride;
            float vf[DPL];
            if constexpr (DPL == 1) {
                vf[0] = tf_h2f(vr[0]);
            } else if constexpr (DPL == 2) {
                const uint32_t vv = *reinterpret_cast<const uint32_t*>(vr);
                vf[0] = tf_h2f(vv);
                vf[1] = tf_h2f(vv >> 16);
            } else {
                const tf_u32x2 vv = *reinterpret_cast<const tf_u32x2*>(vr);
                vf[0] = tf_h2f(vv.x);
                vf[1] = tf_h2f(vv.x >> 16);
                vf[2] = tf_h2f(vv.y);
                vf[3] = tf_h2f(vv.y >> 16);
            }
#pragma unroll
            for (int g = 0; g < GMAX; g++) {
                if (g < G) {
                    const float e = e_lds[wave][g][tt];
#pragma unroll
                    for (int i = 0; i < DPL; i++) o[g][i] += e * vf[i];
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }

    // ---- merge the four wave states (log-sum-exp)
#pragma unroll
    for (int g = 0; g < GMAX; g++) {
        if (g < G) {
            if (lane == 0) {
                m_lds[wave][g] = m[g];
                l_lds[wave][g] = l[g];
            }
#pragma unroll
            for (int i = 0; i < DPL; i++) o_lds[wave][g][lane * DPL + i] = o[g][i];
        }
    }
    __syncthreads();
    const int po = 2 + HD;
    for (int idx = threadIdx.x; idx < G * HD; idx += blockDim.x) {
        const int g = idx / HD, d = idx - g * HD;
        float M = TF_NEG_BIG;
#pragma unroll
        for (int w = 0; w < TF_FLASH_WAVES; w++) M = fmaxf(M, m_lds[w][g]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < TF_FLASH_WAVES; w++) {
            const float a = __expf(m_lds[w][g] - M);
            L += a * l_lds[w][g];
            O += a * o_lds[w][g][d];
        }
        float* base = partial + ((size_t)(kv_h * G + g) * n_split + s) * po;
        if (d == 0) {
            base[0] = M;
            base[1] = L;
        }
        base[2 + d] = O;
    }
}

__global__ __launch_bounds__(256) void tf_flash_reduce_kernel(const float* __restrict__ partial,
                                                              float* __restrict__ out,
                                                              int head_dim, int n_split) {
    const int h = blockIdx.x;
    const int po = 2 + head_dim;
    const float* ph = partial + (size_t)h * n_split * po;
    float M = TF_NEG_BIG;
    for (int s = 0; s < n_split; s++) M = fmaxf(M, ph[(size_t)s * po]);
    for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
        float L = 0.f, acc = 0.f;
        for (int s = 0; s < n_split; s++) {
            const float* b = ph + (size_t)s * po;
            const float a = __expf(b[0] - M);
            L += a * b[1];
            acc += a * b[2 + d];
        }
        out[(size_t)h * head_dim + d] = acc / fmaxf(L, 1e-20f);
    }
}

// ---------------------------------------------------------------- dispatch

template <int HD>
static int tf_flash_launch_hd(const float* q, const uint16_t* k, const uint16_t* v,
                              float* partial, int n_head, int n_kv, int pos0,
                              const int* pos0_dev, int n_split, float scale,
                              tf_stream_t stream) {
    const int G = n_head / n_kv;
    const dim3 grid(n_kv, n_split);
    if (G <= 4)
        hipLaunchKernelGGL((tf_flash_partial_kernel<HD, 4>), grid, dim3(256), 0,
                           tf_stream(stream), q, k, v, partial, n_head, n_kv, pos0, pos0_dev,
                           n_split, scale);
    else if (G <= 8)
        hipLaunchKernelGGL((tf_flash_partial_kernel<HD, 8>), grid, dim3(256), 0,
                           tf_stream(stream), q, k, v, partial, n_head, n_kv, pos0, pos0_dev,
                           n_split, scale);
    else
        return (int)hipErrorInvalidValue;
    return TF_LAUNCH_RESULT();
}

static int tf_flash_partial_any(const float* q, const uint16_t* k, const uint16_t* v,
                                float* partial, int n_head, int n_kv, int head_dim, int pos0,
                                const int* pos0_dev, int n_q, int n_split, float scale,
                                tf_stream_t stream) {
    TF_CHECK_ARG(q && k && v && partial && n_head > 0 && n_kv > 0 && n_head % n_kv == 0);
    TF_CHECK_ARG(n_head / n_kv <= 8 && n_q == 1 && n_split >= 1 && n_split <= 1024);
    TF_CHECK_ARG(pos0_dev || pos0 >= 0);
    TF_CHECK_ARG(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0);
    switch (head_dim) {
    case 64:
        return tf_flash_launch_hd<64>(q, k, v, partial, n_head, n_kv, pos0, pos0_dev, n_split,
                                      scale, stream);
    case 128:
        return tf_flash_launch_hd<128>(q, k, v, partial, n_head, n_kv, pos0, pos0_dev, n_split,
                                       scale, stream);
    case 256:
        return tf_flash_launch_hd<256>(q, k, v, partial, n_head, n_kv, pos0, pos0_dev, n_split,
                                       scale, stream);
    default:
        return (int)hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------- C ABI

extern "C" int tf_flash_decode_partial(const float* q, const uint16_t* k_cache,
                                       const uint16_t* v_cache, float* partial, int n_head,
                                       int n_kv, int head_dim, int pos0, int n_q, int n_split,
                                       float scale, tf_stream_t stream) {
    return tf_flash_partial_any(q, k_cache, v_cache, partial, n_head, n_kv, head_dim, pos0,
                                nullptr, n_q, n_split, scale, stream);
}

extern "C" int tf_flash_decode_partial_d(const float* q, const uint16_t* k_cache,
                                         const uint16_t* v_cache, float* partial, int n_head,
                                         int n_kv, int head_dim, const int* pos0_dev, int n_q,
                                         int n_split, float scale, tf_stream_t stream) {
    TF_CHECK_ARG(pos0_dev != nullptr);
    return tf_flash_partial_any(q, k_cache, v_cache, partial, n_head, n_kv, head_dim, 0,
                                pos0_dev, n_q, n_split, scale, stream);
}

extern "C" int tf_flash_decode_reduce(const float* partial, float* out, int n_head,
                                      int head_dim, int n_split, int n_q, tf_stream_t stream) {
    TF_CHECK_ARG(partial && out && n_head > 0 && head_dim > 0 && n_split >= 1 && n_q == 1);
    const int threads = head_dim <= 64 ? 64 : (head_dim <= 128 ? 128 : 256);
    hipLaunchKernelGGL(tf_flash_reduce_kernel, dim3(n_head), dim3(threads), 0, tf_stream(stream), partial, out, head_dim, n_split);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_flash_decode_n_split(int n_kv, int max_seq) {
    if (n_kv <= 0 || max_seq <= 0) return 8;
    const int cus = tf_device_cus();
    // at least one full 4-wave step (256 tokens) per split; aim for ~2
    // workgroups per CU; multiples of 8 as in the reference's fixed split.
    int by_len = max_seq / (TF_FLASH_WAVES * TF_FLASH_STEP);
    int by_cus = (2 * cus + n_kv - 1) / n_kv;
    int n = by_len < by_cus ? by_len : by_cus;
    n = (n / 8) * 8;
    if (n < 8) n = 8;
    if (n > 1024) n = 1024;
    return n;
}
