// Decode-step glue kernels for gfx950: token embedding row, RMSNorm, NeoX
// RoPE, f32 -> f16 KV append and argmax.  Each has a host-position and a
// device-position ("_d") variant where the reference has one, so that a
// captured HIP graph stays valid while the position advances.
//
// Replaces kernels/embed.cu embed_q{4,6}_k_one[_d] (:51-131), kernels/ops.cu
// rms_norm_f32 (:4-34), rope_neox_f32[_d] (:348-398), copy_kv_f16[_d]
// (:471-504) and argmax_f32 (:573-599).
#include <math.h>

#include "argmax_key.hpp"
#include "dequant.hpp"
#include "tf_common.hpp"
#include "tf_host.hpp"

// ------------------------------------------------------------ embedding

template <int BLOCK_BYTES>
__global__ __launch_bounds__(256) void tf_embed_kernel(const uint8_t* __restrict__ table,
                                                       float* __restrict__ out, int token,
                                                       const int* __restrict__ token_dev,
                                                       int n, int col_bytes) {
    if (token_dev) token = token_dev[0];
    const uint8_t* col = table + (size_t)token * col_bytes;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] = tf_row_value<BLOCK_BYTES>(col, i);
}

// ------------------------------------------------------------ RMSNorm

// out = x * (1/sqrt(mean(x^2) + eps)) * w  (kernels/ops.cu:4-34), one row,
// with the reference's summation order: 256 strided per-thread sums, then a
// halving tree in LDS, so the normalized row is bit-identical to a CPU
// restatement of the same order.
__global__ __launch_bounds__(256) void tf_rms_norm_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          float* __restrict__ out, int n,
                                                          float eps) {
    __shared__ float buf[256];
    float local = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = x[i];
        local = fmaf(v, v, local);  // fused, as under fmad=true
    }
    buf[threadIdx.x] = local;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) buf[threadIdx.x] += buf[threadIdx.x + s];
        __syncthreads();
    }
    const float scale = 1.0f / sqrtf(buf[0] / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) out[i] = x[i] * scale * w[i];
}

// rms_norm_f32 + quantize_q8_global in one launch (kernels/ops.cu:4-34 and
// kernels/gemv.cu:43-65): xb = x * scale * w written in f32, then its Q8
// bytes and scales.  The norm keeps the reference's summation order (256
// strided partial sums, halving tree: levels 128 and 64 through LDS, the
// rest as shfl_down pairs within wave 0, which adds the same pairs); the
// quantization is bit-identical to tf_quantize_q8.
template <int STEPS>  // STEPS * 512 >= n
__global__ __launch_bounds__(256) void tf_norm_quant_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            float* __restrict__ xb,
                                                            int8_t* __restrict__ q8,
                                                            float* __restrict__ d8, int n,
                                                            float eps) {
    __shared__ float buf[256];
    __shared__ float scale_s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Quantization layout: at step k lane L of wave w holds the value pair
    // e0 = 512k + 128w + 2L, e0 + 1 (16 lanes of a DPP row = one 32-group).
    float2 xv[STEPS], wv[STEPS];
#pragma unroll
    for (int k = 0; k < STEPS; k++) {
        const int e0 = 512 * k + 128 * wave + 2 * lane;
        if (512 * k + 128 * wave < n) {
            xv[k] = *reinterpret_cast<const float2*>(x + e0);
            wv[k] = *reinterpret_cast<const float2*>(w + e0);
        }
    }
    // Sum of squares in the reference's order: thread t owns x[t + 256j].
    float local = 0.f;
    {
        float v[2 * STEPS];
#pragma unroll
        for (int j = 0; j < 2 * STEPS; j++) {
            const int i = tid + 256 * j;
            v[j] = i < n ? x[i] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 2 * STEPS; j++)
            if (tid + 256 * j < n) local = fmaf(v[j], v[j], local);  // fused, as under fmad=true
    }
    buf[tid] = local;
    __syncthreads();
    if (tid < 128) buf[tid] += buf[tid + 128];
    __syncthreads();
    if (tid < 64) {
        float v = buf[tid] + buf[tid + 64];
        v += __shfl_down(v, 32, 64);
        v += __shfl_down(v, 16, 64);
        v += __shfl_down(v, 8, 64);
        v += __shfl_down(v, 4, 64);
        v += __shfl_down(v, 2, 64);
        v += __shfl_down(v, 1, 64);
        if (tid == 0) scale_s = 1.0f / sqrtf(v / (float)n + eps);
    }
    __syncthreads();
    const float scale = scale_s;
    const int m = lane & 15;
#pragma unroll
    for (int k = 0; k < STEPS; k++) {
        const int wbase = 512 * k + 128 * wave;
        if (wbase >= n) break;  // n % 128 == 0 here: whole wave spans
        const int e0 = wbase + 2 * lane;
        const float x0 = xv[k].x * scale * wv[k].x;
        const float x1 = xv[k].y * scale * wv[k].y;
        const TfQ8Pair r = tf_q8_pair<false>(x0, x1);
        *reinterpret_cast<float2*>(xb + e0) = make_float2(x0, x1);
        q8[e0] = (int8_t)r.q0;
        q8[e0 + 1] = (int8_t)r.q1;
        if (m == 0) d8[e0 >> 5] = r.d;
    }
}

// ------------------------------------------------------------ RoPE (NeoX)

// Rotates pairs (i, i + hd/2) of every head by pos * theta^(-2i/hd)
// (kernels/ops.cu:348-398).
__global__ __launch_bounds__(64) void tf_rope_neox_kernel(float* __restrict__ x, int head_dim,
                                                          int pos, const int* __restrict__ pos_dev,
                                                          float theta) {
    if (pos_dev) pos = pos_dev[0];
    const int h = blockIdx.x;
    const int half = head_dim / 2;
    float* base = x + (size_t)h * head_dim;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float freq = powf(theta, -2.f * (float)i / (float)head_dim);
        const float ang = (float)pos * freq;
        float s, c;
        sincosf(ang, &s, &c);
        const float x0 = base[i], x1 = base[i + half];
        base[i] = x0 * c - x1 * s;
        base[i + half] = x0 * s + x1 * c;
    }
}

// ------------------------------------------------------------ KV append

__global__ __launch_bounds__(256) void tf_copy_kv_kernel(const float* __restrict__ src,
                                                         uint16_t* __restrict__ cache, int pos,
                                                         const int* __restrict__ pos_dev,
                                                         int stride) {
    if (pos_dev) pos = pos_dev[0];
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < stride) cache[(size_t)pos * stride + i] = tf_f2h_halfup(src[i]);
}

// ------------------------------------------------------------ argmax

// argmax_f32 (kernels/ops.cu:573-599): the reference's winner, ties and
// NaN included, through the 64-bit keys of argmax_key.hpp (every thread
// max-merges the keys of a strided range, then the block merges).
__global__ __launch_bounds__(1024) void tf_argmax_kernel(const float* __restrict__ x, int n,
                                                         int* __restrict__ out_idx) {
    __shared__ unsigned long long part[16];
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const unsigned long long k = tf_argmax_key(x[i], i);
        best = k > best ? k : best;
    }
    best = tf_wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        best = part[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) best = part[w] > best ? part[w] : best;
        out_idx[0] = tf_argmax_key_index(best);
    }
}

// ---------------------------------------------------------------- C ABI

extern "C" int tf_embed_row(const uint8_t* table, int block_bytes, float* out, int token,
                            const int* token_dev, int n_rows, int col_bytes,
                            tf_stream_t stream) {
    // 256-value K-quant blocks cover floor(n_rows / 256) * 256 values (as
    // the reference); 32-value blocks cover n_rows (a multiple of 32)
    const bool k256 = block_bytes == 144 || block_bytes == 210;
    TF_CHECK_ARG(k256 || block_bytes == 34 || block_bytes == 22);
    const int per = k256 ? 256 : 32;
    const int nb = n_rows / per;
    TF_CHECK_ARG(table && out && nb > 0 && (token_dev || token >= 0));
    TF_CHECK_ARG(col_bytes >= nb * block_bytes);
    const int n = nb * per;
    const dim3 grid((n + 255) / 256);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, tf_stream(stream), table, out, token,
                           token_dev, n, col_bytes);
    };
    switch (block_bytes) {
    case 144: go(tf_embed_kernel<144>); break;
    case 210: go(tf_embed_kernel<210>); break;
    case 34: go(tf_embed_kernel<34>); break;
    default: go(tf_embed_kernel<22>); break;
    }
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_rms_norm(const float* x, const float* w, float* out, int n, float eps,
                           tf_stream_t stream) {
    TF_CHECK_ARG(x && w && out && n > 0);
    hipLaunchKernelGGL(tf_rms_norm_kernel, dim3(1), dim3(256), 0, tf_stream(stream), x, w, out, n,
                       eps);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_norm_quant(const float* x, const float* w, float eps, float* xb, int8_t* q8,
                             float* d8, int n, tf_stream_t stream) {
    TF_CHECK_ARG(x && w && xb && q8 && d8 && n > 0 && (n % 128) == 0 && n <= 8192);
    TF_CHECK_ARG(((uintptr_t)x & 7) == 0 && ((uintptr_t)w & 7) == 0 && ((uintptr_t)xb & 7) == 0);
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(1), dim3(256), 0, tf_stream(stream), x, w, xb, q8, d8, n,
                           eps);
    };
    const int steps = (n + 511) / 512;
    if (steps <= 1) launch(tf_norm_quant_kernel<1>);
    else if (steps <= 2) launch(tf_norm_quant_kernel<2>);
    else if (steps <= 4) launch(tf_norm_quant_kernel<4>);
    else if (steps <= 8) launch(tf_norm_quant_kernel<8>);
    else launch(tf_norm_quant_kernel<16>);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_rope_neox(float* x, int n_heads, int head_dim, int pos, const int* pos_dev,
                            float theta, tf_stream_t stream) {
    TF_CHECK_ARG(x && n_heads > 0 && head_dim > 0 && (head_dim & 1) == 0 && (pos_dev || pos >= 0));
    hipLaunchKernelGGL(tf_rope_neox_kernel, dim3(n_heads), dim3(64), 0, tf_stream(stream), x,
                       head_dim, pos, pos_dev, theta);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_copy_kv_f16(const float* src, uint16_t* cache, int pos, const int* pos_dev,
                              int stride, tf_stream_t stream) {
    TF_CHECK_ARG(src && cache && stride > 0 && (pos_dev || pos >= 0));
    hipLaunchKernelGGL(tf_copy_kv_kernel, dim3((stride + 255) / 256), dim3(256), 0,
                       tf_stream(stream), src, cache, pos, pos_dev, stride);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_argmax(const float* x, int n, int* out_idx, tf_stream_t stream) {
    TF_CHECK_ARG(x && n > 0 && out_idx);
    hipLaunchKernelGGL(tf_argmax_kernel, dim3(1), dim3(1024), 0, tf_stream(stream), x, n, out_idx);
    return TF_LAUNCH_RESULT();
}
