// Streaming-read probe: the HBM read rate a kernel with no arithmetic gets
// for a given number of bytes per launch, the floor the batch-1 GEMVs are
// priced against (a GEMV cannot read its weights faster than this).  No
// counterpart in the reference; used by bench.py only.
//
// A grid of `blocks_per_cu` x CUs workgroups of 512 threads reads the
// buffer as 16-byte chunks, U loads in flight per thread per pass, folded
// into one word; a workgroup writes a single word to sink[blockIdx.x] so the
// loads are not dead.  Interleaved: thread t of T reads chunks t, t + T,
// t + 2T, ...; contiguous: workgroup b reads its own run of n / grid chunks,
// 512 consecutive chunks per load instruction of the workgroup.
#include "tf_common.hpp"
#include "tf_host.hpp"

template <int U, bool CONTIG>
__global__ __launch_bounds__(512) void tf_stream_read_kernel(const tf_u32x4* __restrict__ src,
                                                             long long n_chunks,
                                                             uint32_t* __restrict__ sink) {
    long long T = (long long)gridDim.x * 512;
    long long c = (long long)blockIdx.x * 512 + threadIdx.x;
    if (CONTIG) {
        const long long per = (n_chunks + gridDim.x - 1) / gridDim.x;
        const long long b0 = per * blockIdx.x, b1 = b0 + per < n_chunks ? b0 + per : n_chunks;
        src += b0;
        n_chunks = b1 > b0 ? b1 - b0 : 0;
        T = 512;
        c = threadIdx.x;
    }
    uint32_t acc = 0;
    // U loads in flight per pass, every one issued (a chunk past the end
    // reloads chunk c, already on its way, and is not folded in): a tail
    // loop of single loads would pay one memory round trip per chunk
    for (; c < n_chunks; c += U * T) {
        tf_u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const long long cu = c + u * T;
            v[u] = tf_ld16(src + (cu < n_chunks ? cu : c));
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (c + u * T < n_chunks) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    // thread 0's fold stands for the workgroup (every lane's loads are issued
    // regardless: the store is conditional at run time only)
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

extern "C" int tf_stream_read_probe(const void* src, long long n_bytes, uint32_t* sink,
                                    int blocks_per_cu, int depth, int contiguous,
                                    tf_stream_t stream) {
    TF_CHECK_ARG(src && sink && n_bytes >= 16 && n_bytes % 16 == 0 && blocks_per_cu >= 1 &&
                 blocks_per_cu <= 8 && ((uintptr_t)src & 15) == 0);
    const int grid = tf_device_cus() * blocks_per_cu;
    const long long n = n_bytes / 16;
    auto* s = reinterpret_cast<const tf_u32x4*>(src);
    const dim3 g(grid), b(512);
    const hipStream_t st = tf_stream(stream);
    if (contiguous) {
        switch (depth) {
        case 4: hipLaunchKernelGGL((tf_stream_read_kernel<4, true>), g, b, 0, st, s, n, sink); break;
        case 8: hipLaunchKernelGGL((tf_stream_read_kernel<8, true>), g, b, 0, st, s, n, sink); break;
        case 16: hipLaunchKernelGGL((tf_stream_read_kernel<16, true>), g, b, 0, st, s, n, sink); break;
        default: return (int)hipErrorInvalidValue;
        }
    } else {
        switch (depth) {
        case 4: hipLaunchKernelGGL((tf_stream_read_kernel<4, false>), g, b, 0, st, s, n, sink); break;
        case 8: hipLaunchKernelGGL((tf_stream_read_kernel<8, false>), g, b, 0, st, s, n, sink); break;
        case 16: hipLaunchKernelGGL((tf_stream_read_kernel<16, false>), g, b, 0, st, s, n, sink); break;
        default: return (int)hipErrorInvalidValue;
        }
    }
    return TF_LAUNCH_RESULT();
}
