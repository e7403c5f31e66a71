// Allocation-free split-KV flash decode: tf_flash_decode with its two
// workspaces (the split partials and the per-kv-head merge counters) taken
// from a file-scope device array instead of caller buffers, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// Every GPU holds its own copy of `scratch` for the life of the process.
// Its address on the current device comes from hipGetSymbolAddress on the
// first call made with that device current and is kept per device; the
// array's name is never passed to a kernel.  The first call on a device
// also clears the counters with a fill kernel on the caller's stream; every
// flash call leaves them zero again.  Calls that overlap on one GPU share
// the array and race: serialize them (one stream, or events).
#include <mutex>

#include "tf_common.hpp"
#include "tf_host.hpp"

#define TF_NOALLOC_PARTIAL_FLOATS (1u << 20)  // 4 MiB of (m, l, O[hd]) partials
#define TF_NOALLOC_COUNTERS 256u              // one merge counter per kv head

static __device__ __align__(256) unsigned scratch[TF_NOALLOC_PARTIAL_FLOATS + TF_NOALLOC_COUNTERS];

__global__ void tf_noalloc_zero_kernel(unsigned* p, unsigned n) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
unsigned* g_ptr[kMaxDevices] = {};

// The array's address on the current device (set-up on first use).
int scratch_ptr(hipStream_t s, unsigned** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        unsigned* base = static_cast<unsigned*>(p);
        hipLaunchKernelGGL(tf_noalloc_zero_kernel, dim3(1), dim3(256), 0, s,
                           base + TF_NOALLOC_PARTIAL_FLOATS, TF_NOALLOC_COUNTERS);
        e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        g_ptr[dev] = base;
    }
    *out = g_ptr[dev];
    return 0;
}
}  // namespace

extern "C" int tf_flash_decode_noalloc(const float* q, const uint16_t* k_cache,
                                       const uint16_t* v_cache, float* out, int8_t* q8, float* d8,
                                       int n_head, int n_kv, int head_dim, int pos0,
                                       const int* pos0_dev, int n_split, float scale,
                                       tf_stream_t stream) {
    TF_CHECK_ARG(n_head > 0 && n_kv > 0 && head_dim > 0 && n_split >= 1);
    TF_CHECK_ARG((unsigned)n_kv <= TF_NOALLOC_COUNTERS);
    TF_CHECK_ARG((unsigned long long)n_head * n_split * (2 + head_dim) <=
                 TF_NOALLOC_PARTIAL_FLOATS);
    unsigned* base = nullptr;
    const int rc = scratch_ptr(tf_stream(stream), &base);
    if (rc) return rc;
    return tf_flash_decode(q, k_cache, v_cache, reinterpret_cast<float*>(base),
                           base + TF_NOALLOC_PARTIAL_FLOATS, out, q8, d8, n_head, n_kv, head_dim,
                           pos0, pos0_dev, n_split, scale, stream);
}
