// Q8 activation quantize (kernels/gemv.cu:43-65 quantize_q8_global).
//
// One wave64 quantizes two 32-value groups: lanes 0..31 own group 2w and
// lanes 32..63 own group 2w+1.  The group amax is a 5-step xor butterfly
// inside each 32-lane half (max is order-free, so the result is the same as
// the reference's shfl_down tree).
#include "tf_common.hpp"
#include "tf_host.hpp"

__global__ __launch_bounds__(256) void tf_quantize_q8_kernel(
    const float* __restrict__ x, int8_t* __restrict__ q8,
    float* __restrict__ d8, int n_groups) {
    const int lane = threadIdx.x & 63;
    const int g = (blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    const bool live = g < n_groups;
    const float xi = live ? x[g * 32 + (lane & 31)] : 0.f;
    float amax = tf_group32_max(fabsf(xi));
    const float d = amax * (1.0f / 127.0f);
    if (live) {
        q8[g * 32 + (lane & 31)] = (int8_t)tf_q8_value(xi, amax, d);
        if ((lane & 31) == 0) d8[g] = d;
    }
}

extern "C" int tf_quantize_q8(const float* x, int8_t* q8, float* d8,
                              int n_rows, tf_stream_t stream) {
    TF_CHECK_ARG(x && q8 && d8 && n_rows > 0 && (n_rows % 32) == 0);
    const int groups = n_rows / 32;
    const int blocks = (groups + 7) / 8;
    hipLaunchKernelGGL(tf_quantize_q8_kernel, dim3(blocks), dim3(256), 0,
                       tf_stream(stream), x, q8, d8, groups);
    return TF_LAUNCH_RESULT();
}
