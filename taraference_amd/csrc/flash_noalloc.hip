// Allocation-free split-KV flash decode: tf_flash_decode with its split
// partials taken from a file-scope device array instead of a caller buffer,
// for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// Every GPU holds its own copy of `scratch` for the life of the process.
// Its address on the current device comes from hipGetSymbolAddress on the
// first call made with that device current and is kept per device; the
// array's name is never passed to a kernel.  The set-up enqueues nothing,
// so a first call made under stream capture records only the flash
// kernels.  Every call overwrites the partials it reads (nothing needs to
// start at zero).  Calls that overlap on one GPU share the array and race:
// serialize them (one stream, or events).
#include <mutex>

#include "tf_common.hpp"
#include "tf_host.hpp"

#define TF_NOALLOC_PARTIAL_FLOATS (1u << 20)  // 4 MiB of (m, l, O[hd]) partials

static __device__ __align__(256) float scratch[TF_NOALLOC_PARTIAL_FLOATS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_ptr[kMaxDevices] = {};

// The array's address on the current device (set-up on first use).
int scratch_ptr(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_ptr[dev] = static_cast<float*>(p);
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
    TF_CHECK_ARG((unsigned long long)n_head * n_split * (2 + head_dim) <=
                 TF_NOALLOC_PARTIAL_FLOATS);
    float* base = nullptr;
    const int rc = scratch_ptr(&base);
    if (rc) return rc;
    return tf_flash_decode(q, k_cache, v_cache, base, nullptr, out, q8, d8, n_head, n_kv,
                           head_dim, pos0, pos0_dev, n_split, scale, stream);
}
