// Persistent decode step for gfx950: one launch runs a whole batch-1 greedy
// decode step (embedding, every layer, lm_head and argmax) of a dense
// Qwen2-style Q4_K_M model.  It performs the same operator sequence as the
// multi-launch fused path (model.cpp step_fused), which restates
// cuda/forward.rs:73-264 and cuda/layer.rs:99-709, 1210-1456, 2125-2259:
//
//   per layer: [norm + Q8 + QKV + RoPE + K/V append] | [split-KV attention
//   with its log-sum-exp merge] | [wo, residual] | [norm + Q8 + gate/up +
//   SiLU] | [Q8 + down, residual];  then [norm + Q8 + lm_head + argmax].
//
// Why one launch: at batch 1 every stage streams a few MB of weights, so a
// launch per stage pays the launch gap plus the ramp of its first HBM
// requests each time.  Here one workgroup per CU stays resident and the
// stages are separated by grid barriers.  The weights a wave needs for its
// first task of the next stage do not depend on the barrier, so each wave
// issues those loads BEFORE it waits: HBM keeps streaming across every
// dependency.
//
// Cross-XCD coherence.  The eight XCDs have private L2s.  Everything a stage
// produces for another workgroup (q, K/V rows, attention partials and
// output, x, h, argmax keys, barrier words) is written with device-scope
// atomic stores and read with device-scope atomic loads, which bypass the
// non-coherent L2 state; each thread drains its stores (s_waitcnt) before
// its workgroup signals a barrier.  No L2 write-back fence is needed, which
// is what makes a barrier cost about 2 us instead of 7-15 us.  Data written by
// earlier launches (weights, K/V rows below the current position) is read
// with ordinary loads.
//
// Barrier: flag array.  Workgroup b stores the epoch into its own 128-byte
// line; workgroup 0 polls all lines (one thread each) and then stores the
// epoch into the release word that everybody polls.  Epochs grow
// monotonically across launches (a generation word advances once per
// launch), compared with wrap-around arithmetic.  Every spin is bounded: on a
// time-out the workgroup raises the abort word and the error word and
// returns, and every other wait sees the abort word and returns too, so the
// grid always drains.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "argmax_key.hpp"
#include "lds_dma.hpp"
#include "decode_persistent.hpp"
#include "dequant.hpp"
#include "q4k.hpp"
#include "q6k.hpp"
#include "tf_host.hpp"

// The argument and layer tables are copied into LDS when a launch starts and
// read from there (address space 3).  A table field read from global memory
// inside a stage would be a vector load, and vector loads complete in
// order: it would wait for every weight load the wave had issued before it,
// i.e. for the whole prefetch of the stage.
#define TF_LAS __attribute__((address_space(3)))
typedef const TF_LAS TfPArgs TfPA;
typedef const TF_LAS TfPLayer TfPL;
#define TF_P_MAX_LAYERS 64
static_assert(sizeof(TfPArgs) % 4 == 0 && sizeof(TfPLayer) % 4 == 0, "tables copy as words");
__shared__ TfPArgs tf_p_args;
__shared__ TfPLayer tf_p_layers[TF_P_MAX_LAYERS];

// The dynamic LDS of the kernel, named at file scope so that every stage
// function addresses it as LDS.
extern __shared__ __align__(16) uint8_t tf_p_lds[];
__shared__ int tf_p_ok, tf_p_flag;  // tf_p_flag: sticky per-launch abort
__shared__ int tf_p_last;

#define TF_P_THREADS 512
#define TF_P_WAVES (TF_P_THREADS / 64)
#define TF_SPIN_LIMIT (1 << 20)
#define TF_P_TILE 64
#define TF_P_HD 128
#define TF_P_NEG_BIG (-1e30f)

// ------------------------------------------------------ coherent access

__device__ __forceinline__ TfPL& tf_p_layer(TfPA& a, int li) {
    return ((TfPL*)tf_p_layers)[li];
}

__device__ __forceinline__ unsigned tf_ldu(const unsigned* p) {
    return __hip_atomic_load((TF_GAS unsigned*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tf_stu(unsigned* p, unsigned v) {
    __hip_atomic_store((TF_GAS unsigned*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float tf_ldc(const float* p) {
    return __hip_atomic_load((TF_GAS float*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tf_stc(float* p, float v) {
    __hip_atomic_store((TF_GAS float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long tf_ldc64(const void* p) {
    return __hip_atomic_load((TF_GAS unsigned long long*)p, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tf_stc64(void* p, unsigned long long v) {
    __hip_atomic_store((TF_GAS unsigned long long*)p, v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 tf_ldc2(const float* p) {
    const unsigned long long v = tf_ldc64(p);
    return make_float2(__uint_as_float((unsigned)v), __uint_as_float((unsigned)(v >> 32)));
}
__device__ __forceinline__ tf_u32x4 tf_ldc16(const void* p) {
    const unsigned long long a = tf_ldc64(p);
    const unsigned long long b = tf_ldc64(reinterpret_cast<const uint8_t*>(p) + 8);
    return tf_u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}
__device__ __forceinline__ void tf_stc_h(uint16_t* p, uint16_t v) {
    __hip_atomic_store((TF_GAS uint16_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------ lane ids
//
// threadIdx.x through an empty volatile asm: the compiler cannot hoist what
// is derived from it out of the layer loop, so each stage's lane geometry
// is recomputed where it is used instead of staying live (in registers)
// across the whole loop.
__device__ __forceinline__ int tf_p_tid() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int tf_p_wid() {
    return (tf_p_tid() >> 6) * (int)gridDim.x + (int)blockIdx.x;
}

// ------------------------------------------------ flagged vectors
//
// Stage outputs travel as 64-bit words: low half the value bits, high half a
// tag naming the (launch, layer, vector) that wrote it.  A producer stores
// each element with one 64-bit device-scope atomic store; a consumer loads
// the words it needs and retries the ones whose tag is not yet the expected
// one.  The 64-bit access is single-copy atomic, so a matching tag
// guarantees the value beside it; no barrier, fence or store drain separates
// the stages.  Each vector is double-buffered by layer parity, and every
// workgroup both reads a vector and contributes to the vectors computed from
// it, so a buffer is not rewritten before every reader is done with it.
// Tags grow with the launch generation; the runtime zeroes the buffers
// (tag 0, never expected) whenever it resets the generation.

// lm_head tasks in flight per wave (3 / 4 / 5: 1019 / 1020 / 1013 tok/s) and the
// all-wave polls' s_sleep between rounds (2 / 4 / 8: no measurable change)
#ifndef TF_P_HEAD_D
#define TF_P_HEAD_D 4
#endif
#ifndef TF_P_SLEEP
#define TF_P_SLEEP 4
#endif

enum TfPKind {
    TF_PK_XA = 0, TF_PK_XB = 1, TF_PK_Q = 2, TF_PK_KV = 3, TF_PK_O = 4, TF_PK_H = 5, TF_PK_PART = 6,
    TF_PK_HX = 7
};

__device__ __forceinline__ unsigned tf_p_tag(unsigned tb, int li, int kind) {
    return tb + 8u * (unsigned)li + (unsigned)kind + 1u;
}

__device__ __forceinline__ void tf_p_put(unsigned long long* p, uint32_t bits, unsigned tag) {
    tf_stc64(p, (unsigned long long)bits | ((unsigned long long)tag << 32));
}
__device__ __forceinline__ void tf_p_putf(unsigned long long* p, float v, unsigned tag) {
    tf_p_put(p, __float_as_uint(v), tag);
}

__device__ __forceinline__ void tf_p_abort(TfPA& a) {
    tf_stu(a.bar + TF_BAR_ABORT, 1u);
    __hip_atomic_fetch_or((TF_GAS int*)a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stage timeline (diagnostics): stage k of this workgroup started (0), had
// its activation staged (2) and finished (3).
// The stamps collect in LDS (a global store here would hold up the wave's
// next memory wait) and are copied out at the end of the launch.
__shared__ unsigned long long tf_p_tstamp[(5 * TF_P_MAX_LAYERS + 1) * 4];

__device__ __forceinline__ void tf_p_stamp(TfPA& a, int k, int which, int who = 0) {
    if (a.trace && tf_p_tid() == who) tf_p_tstamp[k * 4 + which] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ void tf_p_trace_flush(TfPA& a) {
    if (!a.trace) return;
    __syncthreads();
    for (int i = tf_p_tid(); i < (5 * a.n_layer + 1) * 4; i += TF_P_THREADS)
        a.trace[((size_t)(i >> 2) * gridDim.x + blockIdx.x) * 4 + (i & 3)] = tf_p_tstamp[i];
}

// dst(i, bits) for i < n once word i of src carries `tag`; threads r, r + R,
// r + 2R, ... of a group of R threads (r = rank), P passes of K words per
// thread (K R P >= n, checked: a longer vector aborts the launch).  The
// passes are unrolled and every load is issued unconditionally (past-the-end
// words reload word 0): a load under a branch, or a loop back edge, makes
// the compiler drain all loads in flight (the weight prefetch included)
// before issuing the next one.  WG: must be called by every thread of the
// workgroup; returns false (everywhere) if the wait timed out or the launch
// was aborted.  !WG: called by the R threads alone, no barrier; a time-out
// or abort sets tf_p_flag, which the caller reads after its next barrier.
// Two flagged vectors polled as one: words [0, n0) of a (tag ta), then b (tag tb).
struct TfPSplitSrc {
    const unsigned long long *a, *b;
    int n0;
    unsigned ta, tb;
};
__device__ __forceinline__ unsigned long long tf_p_src_ld(const unsigned long long* p, int i) {
    return tf_ldc64(p + i);
}
__device__ __forceinline__ unsigned tf_p_src_tag(const unsigned long long*, unsigned tag, int) {
    return tag;
}
__device__ __forceinline__ unsigned long long tf_p_src_ld(const TfPSplitSrc& s, int i) {
    return tf_ldc64(i < s.n0 ? s.a + i : s.b + (i - s.n0));
}
__device__ __forceinline__ unsigned tf_p_src_tag(const TfPSplitSrc& s, unsigned, int i) {
    return i < s.n0 ? s.ta : s.tb;
}

template <int K, int P, class Dst, bool WG = true, class Src = const unsigned long long*>
__device__ __forceinline__ bool tf_p_poll(Dst dst, Src src, int n, unsigned tag, int rank, int R,
                                          TfPA& a) {
    int bad = n > K * R * P;
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int i0 = rank + p * K * R;
        unsigned long long v[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = i0 + k * R;
            v[k] = tf_p_src_ld(src, i < n ? i : 0);
        }
        for (int spins = 0; !bad;) {
            bool miss = false;
#pragma unroll
            for (int k = 0; k < K; k++)
                miss |= (unsigned)(v[k] >> 32) != tf_p_src_tag(src, tag, i0 + k * R) && i0 + k * R < n;
            if (!miss) break;
            if (++spins > TF_SPIN_LIMIT || ((spins & 15) == 0 && tf_ldu(a.bar + TF_BAR_ABORT))) {
                bad = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(TF_P_SLEEP);
#pragma unroll
            for (int k = 0; k < K; k++) {
                const int i = i0 + k * R;
                v[k] = tf_p_src_ld(src, i < n ? i : 0);
            }
        }
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = i0 + k * R;
            if (i < n) dst(i, (uint32_t)v[k]);
        }
    }
    if (bad) {
        tf_p_abort(a);
        tf_p_flag = 1;
    }
    if constexpr (!WG) return !bad;
    __syncthreads();
    const bool ok = tf_p_flag == 0;
    __syncthreads();
    return ok;
}

// ------------------------------------------------- activation staging
//
// The LDS image has the layout of tf_act_view (stage.hpp): q8 | d8 | ds |
// s16 | xf | xs16 for nb super-blocks.  The staging is bit-identical to
// tf_quantize_q8 / tf_norm_quant / tf_stage_act: the Q8 of a 32-value group
// depends only on its values (d = amax fl(1/127), q = rint_even(x / d) with
// an IEEE-exact quotient, kernels/gemv.cu:16-65); integer sums are exact in
// any order; the f32 16-value sums keep the pairwise tree
// ((x0+x1)+(x2+x3))+((x4+x5)+(x6+x7)) + ... of the reference staging; and
// the RMS scale keeps the reference's summation order (below).
//
// Lane map: eight lanes per 32-value group, lane j of the group holding
// values 4j .. 4j+3, so every thread of the workgroup stages four values per
// step and every group reduction is three DPP steps.

// Where a quantizer records its input and output when the launch keeps a Q8
// record (TfPArgs::q8x); all nullptr otherwise.
struct TfPQ8Rec {
    float* x;
    int8_t* q;
    float* d;
};

// REC: the kernel instantiation that keeps the record (production launches
// compile it out).
template <bool REC>
__device__ __forceinline__ TfPQ8Rec tf_p_q8rec(TfPA& a, int li, int site, bool on = true) {
    if (!REC || !a.q8x || !on) return TfPQ8Rec{nullptr, nullptr, nullptr};
    const size_t off = ((size_t)li * 4 + site) * (size_t)a.q8n;
    return TfPQ8Rec{a.q8x + off, a.q8q + off, a.q8d + off / 32};
}

// Q8 of four values held by one lane of an 8-lane group (lane j = lane & 7
// holds values 4 j .. 4 j + 3 of the 32): per value the rule of
// tf_q8_value_r, with the IEEE quotients of a lane taken in one branch.  s_half: int sum over the lane's 16-value
// half (lanes 0-3 or 4-7), s_other: the other half's; f_half the f32 sum of
// the half in the pairwise tree ((x0 + x1) + (x2 + x3)) + ... .
struct TfQ8Quad {
    int q[4];
    float d;
    int s_half, s_other;
    float f_half;
};

template <bool F32>
__device__ __forceinline__ TfQ8Quad tf_q8_g8(const float (&x)[4]) {
    TfQ8Quad r;
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) am = fmaxf(am, fabsf(x[i]));
    uint32_t u = __builtin_bit_cast(uint32_t, am);  // magnitudes order as unsigned ints
    u = max(u, (uint32_t)tf_dppi<TF_DPP_QUAD_1032>((int)u));
    u = max(u, (uint32_t)tf_dppi<TF_DPP_QUAD_2301>((int)u));
    u = max(u, (uint32_t)tf_dppi<TF_DPP_ROW_HALF_MIRROR>((int)u));
    const float amax = __builtin_bit_cast(float, u);
    r.d = amax * (1.0f / 127.0f);
    const float rcp = __builtin_amdgcn_rcpf(r.d);
    // as tf_q8_value_r: the product is exact enough away from a .5 tie; near one
    // (rare) the IEEE quotient decides
    float y[4];
    bool rk[4], any = false;
    const bool tiny = !(r.d >= 1.17549435e-38f);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        y[i] = x[i] * rcp;
        const float fr = fabsf(y[i] - __builtin_truncf(y[i]));
        rk[i] = tiny || fabsf(fr - 0.5f) < 6.103515625e-05f;
        any |= rk[i];
    }
    if (any) {
        const float dd = amax == 0.f ? 1.f : r.d;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (rk[i]) y[i] = x[i] / dd;
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.q[i] = amax == 0.f ? 0 : (int)__builtin_rintf(y[i]);
        s += r.q[i];
    }
    s += tf_dppi<TF_DPP_QUAD_1032>(s);
    r.s_half = s + tf_dppi<TF_DPP_QUAD_2301>(s);
    r.s_other = tf_dppi<TF_DPP_ROW_HALF_MIRROR>(r.s_half);  // lane 7 - j: the other half
    r.f_half = 0.f;
    if (F32) {
        const float t4 = (x[0] + x[1]) + (x[2] + x[3]);
        const float t8 = t4 + tf_dpp<TF_DPP_QUAD_1032>(t4);
        r.f_half = t8 + tf_dpp<TF_DPP_QUAD_2301>(t8);
    }
    return r;
}

// The 4 norm weights per step a thread applies in tf_p_stage8b (values
// 4 tid + 4 TF_P_THREADS step .. + 3), loaded before the stage's weights.
template <int NS>
__device__ __forceinline__ void tf_p_norm_wload4(const float* w, int n, float (&r)[NS][4]) {
#pragma unroll
    for (int st = 0; st < NS; st++) {
        const int e0 = 4 * tf_p_tid() + 4 * TF_P_THREADS * st;
        const tf_u32x4 v = tf_ld16(w + (e0 < n ? e0 : 0));
        r[st][0] = __uint_as_float(v.x);
        r[st][1] = __uint_as_float(v.y);
        r[st][2] = __uint_as_float(v.z);
        r[st][3] = __uint_as_float(v.w);
    }
}

// The activation image of the n = 256 nb values src[0 .. n) in LDS, eight
// lanes per group (tf_q8_g8): every thread of the workgroup takes four
// values per step (NS steps cover 4 TF_P_THREADS NS values).
// Ends with a workgroup barrier.
template <bool F32, bool NORM, int NS>
__device__ __forceinline__ void tf_p_stage8b(uint8_t* lds, int nb, const float* src, float scale,
                                             const float (&w)[NS][4],
                                             TfPQ8Rec rec = TfPQ8Rec{nullptr, nullptr, nullptr}) {
    int8_t* q8s = reinterpret_cast<int8_t*>(lds);
    float* d8s = reinterpret_cast<float*>(lds + TF_Q8_LDS_BYTES(nb));
    float* dss = d8s + nb * 8;
    int32_t* s16 = reinterpret_cast<int32_t*>(dss + nb * 8);
    float* xf = reinterpret_cast<float*>(s16 + nb * 16);
    float* xs16 = xf + nb * 256;
    const int n = nb * 256;
    const int tid = tf_p_tid(), j = tid & 7;
#pragma unroll
    for (int st = 0; st < NS; st++) {
        const int e0 = 4 * tid + 4 * TF_P_THREADS * st;
        if (4 * TF_P_THREADS * st >= n) break;  // workgroup-uniform
        const int e = e0 < n ? e0 : 0;
        const int g = e >> 5;
        const float4 a = *reinterpret_cast<const float4*>(src + e);
        float x[4] = {a.x, a.y, a.z, a.w};
        if (NORM) {
#pragma unroll
            for (int i = 0; i < 4; i++) x[i] = x[i] * scale * w[st][i];
        }
        const TfQ8Quad r = tf_q8_g8<F32>(x);
        if (e0 < n) {
            uint32_t b = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) b |= (uint32_t)(r.q[i] & 0xff) << (8 * i);
            *reinterpret_cast<uint32_t*>(q8s + tf_q8_pad(e)) = b;
            if ((j & 3) == 0) {
                s16[2 * g + (j >> 2)] = r.s_half;
                if (F32) xs16[2 * g + (j >> 2)] = r.f_half;
            }
            if (j == 0) {
                d8s[g] = r.d;
                dss[g] = r.d * (float)(r.s_half + r.s_other);
            }
            if (F32 && NORM) *reinterpret_cast<float4*>(xf + e) = make_float4(x[0], x[1], x[2], x[3]);
            if (rec.x) {  // workgroup-uniform (the Q8 record)
                *reinterpret_cast<float4*>(rec.x + e) = make_float4(x[0], x[1], x[2], x[3]);
                *reinterpret_cast<uint32_t*>(rec.q + e) = b;
                if (j == 0) rec.d[g] = r.d;
            }
        }
    }
    __syncthreads();
}

// LDS word carrying the RMS scale from wave 0 to the others.
__shared__ float tf_p_rms;

// 1 / sqrt(mean(x^2) + eps) of the n values x[0 .. n) in LDS, computed by
// each wave on its own in the reference's order (kernels/ops.cu:4-34):
// partial t (t < 256) = fused square-accumulate of x[t], x[t + 256], ... in
// turn; then red[t] = p(t) + p(t + 128) (t < 128), v = red[t] + red[t + 64]
// (t < 64), then the shift-down tree over 32, 16, ..., 1 -- the same
// additions tf_norm_quant performs through LDS.
// The four partials of a lane advance together, four terms at a time with
// their LDS reads issued first; a padded term adds fmaf(0, 0, p) = p
// exactly (p >= +0), so the value is that of the plain per-partial loop.
__device__ __forceinline__ float tf_p_rms_scale(const float* x, int n, float eps) {
    const int lane = tf_p_tid() & 63;
    const int nj = n / 256;
    float p[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < nj; j0 += 4) {
        float v[4][4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const int j = j0 + jj < nj ? j0 + jj : nj - 1;
#pragma unroll
            for (int c = 0; c < 4; c++) v[jj][c] = x[lane + 64 * c + 256 * j];
        }
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float t = j0 + jj < nj ? v[jj][c] : 0.f;
                p[c] = fmaf(t, t, p[c]);
            }
    }
    float v = (p[0] + p[2]) + (p[1] + p[3]);
    v += __shfl_down(v, 32, 64);
    v += __shfl_down(v, 16, 64);
    v += __shfl_down(v, 8, 64);
    v += __shfl_down(v, 4, 64);
    v += __shfl_down(v, 2, 64);
    v += __shfl_down(v, 1, 64);
    v = tf_readlane(v, 0);
    return 1.0f / sqrtf(v / (float)n + eps);
}

// The RMSNorm input polled by every wave (K words per thread) into raw; wave 0
// then forms the scale from LDS in the reference's order (tf_p_rms_scale)
// into tf_p_rms.  Every thread calls it; false (everywhere): aborted.  The
// caller's next barrier publishes tf_p_rms.  (A poll by wave 0 alone, forming
// the squares while it polls, saw the vector 0.35-0.45 us later.)
template <int K>
__device__ __forceinline__ bool tf_p_poll_rms_wg(TfPA& a, float* raw,
                                                 const unsigned long long* src, int n,
                                                 unsigned tag, float eps) {
    if (!tf_p_poll<K, 1>([&](int i, uint32_t b) { raw[i] = __uint_as_float(b); }, src, n, tag,
                         tf_p_tid(), TF_P_THREADS, a))
        return false;
    if ((tf_p_tid() >> 6) == 0) {
        const float sc = tf_p_rms_scale(raw, n, eps);
        if (tf_p_tid() == 0) tf_p_rms = sc;
    }
    return true;
}


// Raw (unnormalized) row of a norm stage: an LDS area after the image.
__device__ __forceinline__ float* tf_p_raw(uint8_t* lds, int nbE) {
    return reinterpret_cast<float*>(lds + tf_act_lds_bytes(nbE, true));
}

// ------------------------------------------------------------ lane map

struct TfPLane {
    int lane, t, slot, unit, sir;
};
template <int SPR>
__device__ __forceinline__ TfPLane tf_p_lane() {
    TfPLane l;
    l.lane = tf_p_tid() & 63;
    l.t = l.lane & 3;
    l.slot = l.lane >> 2;
    l.unit = l.slot / SPR;
    l.sir = l.slot % SPR;
    return l;
}

// --------------------------------------------- QKV + RoPE + K/V append
//
// Task map as tf_fused_qkv_kernel (decode_fused.hip): Q/K rows in RoPE
// pairs (i, i + hd/2) of one head, then V rows.

// cos/sin of the NeoX rotation angles at this launch's position
// (kernels/ops.cu:374-398: freq = theta^(-2i/hd), angle = pos * freq),
// computed once per launch into tf_p_rope_cs[2i] = cos, [2i+1] = sin.
__shared__ float tf_p_rope_cs[TF_P_HD];

__device__ __forceinline__ void tf_p_rope_table(int hd, int pos, float theta) {
    const int i = tf_p_tid();
    if (i < hd / 2) {
        const float freq = powf(theta, -2.f * (float)i / (float)hd);
        const float ang = (float)pos * freq;
        float s, c;
        sincosf(ang, &s, &c);
        tf_p_rope_cs[2 * i] = c;
        tf_p_rope_cs[2 * i + 1] = s;
    }
}

__device__ __forceinline__ void tf_p_rope(float x0, float x1, int i, float& y0, float& y1) {
    const float2 cs = *reinterpret_cast<const float2*>(tf_p_rope_cs + 2 * i);
    y0 = x0 * cs.x - x1 * cs.y;
    y1 = x0 * cs.y + x1 * cs.x;
}

// Flagged new K/V row: per kv head, its K row (head_dim values) then its V row.
__device__ __forceinline__ int tf_p_kv_k(int idx, int hd) { return (idx / hd) * 2 * hd + idx % hd; }

template <int SPR, int IT>
struct TfPQkvRegs {
    TfQ4kRow<IT> a, b;
    TfQ6kPart v[IT];
    float b0, b1;  // the biases of the task's rows (loaded with the weights)
};

struct TfPQkvGeo {
    int n_q, n_k, n_v, n_pairs, pair_tasks, n_tasks;
};

template <int SPR>
__device__ __forceinline__ TfPQkvGeo tf_p_qkv_geo(TfPA& a) {
    constexpr int UNITS = 16 / SPR, PPT = UNITS >= 2 ? UNITS / 2 : 1;
    TfPQkvGeo g;
    g.n_q = a.H * a.HD;
    g.n_k = a.KV * a.HD;
    g.n_v = g.n_k;
    g.n_pairs = (g.n_q + g.n_k) / 2;
    g.pair_tasks = (g.n_pairs + PPT - 1) / PPT;
    g.n_tasks = g.pair_tasks + (g.n_v + UNITS - 1) / UNITS;
    return g;
}

template <int SPR, int IT>
__device__ __forceinline__ void tf_p_qkv_load(TfPA& a, TfPL& L, int task,
                                              TfPQkvRegs<SPR, IT>& r) {
    constexpr int UNITS = 16 / SPR, PPT = UNITS >= 2 ? UNITS / 2 : 1;
    const TfPQkvGeo g = tf_p_qkv_geo<SPR>(a);
    const TfPLane ln = tf_p_lane<SPR>();
    const int nb = a.E / 256, hd = a.HD, half = hd / 2;
    if (task >= g.n_tasks) return;
    if (task < g.pair_tasks) {
        if constexpr (UNITS >= 2) {
            const int pair = task * PPT + ln.unit / 2, member = ln.unit & 1;
            const bool valid = pair < g.n_pairs;
            const int p = valid ? pair : 0;
            const int row = (p / half) * hd + p % half + member * half;
            const uint8_t* col = row < g.n_q ? L.wq + (size_t)row * L.cb_qk
                                             : L.wk + (size_t)(row - g.n_q) * L.cb_qk;
            tf_q4k_row_load<SPR, IT>(col, valid, 0, nb, ln.sir, ln.t, r.a);
            const float* bias = row < g.n_q ? L.bq : L.bk;
            if (bias) r.b0 = tf_gld(bias + (row < g.n_q ? row : row - g.n_q));
        } else {
            const int r0 = (task / half) * hd + task % half, r1 = r0 + half;
            const bool is_q = r0 < g.n_q;
            const uint8_t* base = is_q ? L.wq : L.wk;
            const int off = is_q ? 0 : g.n_q;
            tf_q4k_row_load<SPR, IT>(base + (size_t)(r0 - off) * L.cb_qk, true, 0, nb, ln.sir, ln.t,
                                     r.a);
            tf_q4k_row_load<SPR, IT>(base + (size_t)(r1 - off) * L.cb_qk, true, 0, nb, ln.sir, ln.t,
                                     r.b);
            const float* bias = is_q ? L.bq : L.bk;
            if (bias) {
                r.b0 = tf_gld(bias + (r0 - off));
                r.b1 = tf_gld(bias + (r1 - off));
            }
        }
    } else {
        const int j = (task - g.pair_tasks) * UNITS + ln.unit;
        const bool valid = j < g.n_v;
        const uint8_t* col = L.wv + (size_t)(valid ? j : 0) * L.cb_v;
        if (L.bv) r.b0 = tf_gld(L.bv + (valid ? j : 0));
        if (L.v_q6k) {
#pragma unroll
            for (int i = 0; i < IT; i++) {
                const int sb = ln.sir + i * SPR;
                if (valid && sb < nb) tf_q6k_load_r(col + (size_t)sb * 210, ln.t, r.v[i]);
            }
        } else {
            tf_q4k_row_load<SPR, IT>(col, valid, 0, nb, ln.sir, ln.t, r.a);
        }
    }
}

template <int SPR, int IT>
__device__ __forceinline__ void tf_p_qkv_task(TfPA& a, TfPL& L, int task, int pos,
                                              const TfAct& x, TfPQkvRegs<SPR, IT>& r,
                                              unsigned long long* fq, unsigned long long* fkv,
                                              unsigned tq, unsigned tkv) {
    constexpr int UNITS = 16 / SPR, PPT = UNITS >= 2 ? UNITS / 2 : 1;
    const TfPQkvGeo g = tf_p_qkv_geo<SPR>(a);
    const TfPLane ln = tf_p_lane<SPR>();
    const int nb = a.E / 256, hd = a.HD, half = hd / 2;
    const int stride = a.KV * hd;
    const bool lead = (ln.lane & (4 * SPR - 1)) == 0;
    if (task < g.pair_tasks) {
        if constexpr (UNITS >= 2) {
            const int pair = task * PPT + ln.unit / 2, member = ln.unit & 1;
            const bool valid = pair < g.n_pairs;
            const int p = valid ? pair : 0;
            const int i = p % half;
            const int row = (p / half) * hd + i + member * half;
            const bool is_q = row < g.n_q;
            float acc = tf_q4k_row_partial<SPR, IT>(r.a, valid, 0, nb, ln.sir, ln.t, x);
            acc = tf_group_sum<4 * SPR>(acc);
            const float* bias = is_q ? L.bq : L.bk;
            if (valid && bias) acc += r.b0;
            const float other = __shfl(acc, ln.lane ^ (4 * SPR), 64);
            const float x0 = member == 0 ? acc : other;
            const float x1 = member == 0 ? other : acc;
            float y0, y1;
            tf_p_rope(x0, x1, i, y0, y1);
            const float y = member == 0 ? y0 : y1;
            if (valid && lead) {
                if (is_q) {
                    tf_p_putf(fq + row, y, tq);
                } else {
                    const uint16_t hv = tf_f2h_halfup(y);
                    *(TF_GAS uint16_t*)(L.k_cache + (size_t)pos * stride + (row - g.n_q)) = hv;
                    tf_p_put(fkv + tf_p_kv_k(row - g.n_q, hd), hv, tkv);
                }
            }
        } else {
            const int i = task % half;
            const int r0 = (task / half) * hd + i, r1 = r0 + half;
            const bool is_q = r0 < g.n_q;
            const int off = is_q ? 0 : g.n_q;
            float x0 = tf_group_sum<64>(tf_q4k_row_partial<SPR, IT>(r.a, true, 0, nb, ln.sir, ln.t, x));
            float x1 = tf_group_sum<64>(tf_q4k_row_partial<SPR, IT>(r.b, true, 0, nb, ln.sir, ln.t, x));
            const float* bias = is_q ? L.bq : L.bk;
            if (bias) {
                x0 += r.b0;
                x1 += r.b1;
            }
            float y0, y1;
            tf_p_rope(x0, x1, i, y0, y1);
            if (ln.lane == 0) {
                if (is_q) {
                    tf_p_putf(fq + r0, y0, tq);
                    tf_p_putf(fq + r1, y1, tq);
                } else {
                    const uint16_t h0 = tf_f2h_halfup(y0), h1 = tf_f2h_halfup(y1);
                    *(TF_GAS uint16_t*)(L.k_cache + (size_t)pos * stride + (r0 - off)) = h0;
                    *(TF_GAS uint16_t*)(L.k_cache + (size_t)pos * stride + (r1 - off)) = h1;
                    tf_p_put(fkv + tf_p_kv_k(r0 - off, hd), h0, tkv);
                    tf_p_put(fkv + tf_p_kv_k(r1 - off, hd), h1, tkv);
                }
            }
        }
    } else {
        const int j = (task - g.pair_tasks) * UNITS + ln.unit;
        const bool valid = j < g.n_v;
        float acc = 0.f;
        if (L.v_q6k) {
#pragma unroll
            for (int i = 0; i < IT; i++) {
                const int sb = ln.sir + i * SPR;
                if (valid && sb < nb) acc += tf_q6k_f32_part_dot(r.v[i], ln.t, sb, x);
            }
            acc = tf_group_sum<4 * SPR>(acc);
        } else {
            acc = tf_group_sum<4 * SPR>(tf_q4k_row_partial<SPR, IT>(r.a, valid, 0, nb, ln.sir, ln.t, x));
        }
        if (valid && lead) {
            if (L.bv) acc += r.b0;
            const uint16_t hv = tf_f2h_halfup(acc);
            *(TF_GAS uint16_t*)(L.v_cache + (size_t)pos * stride + j) = hv;
            tf_p_put(fkv + tf_p_kv_k(j, hd) + hd, hv, tkv);
        }
    }
}

// ------------------------------------------------------ row GEMV stages

template <int IT, bool Q6>
using TfPRow = std::conditional_t<Q6, TfQ6kRow<IT>, TfQ4kRow<IT>>;

template <int SPR, int IT, bool Q6>
__device__ __forceinline__ void tf_p_rows_load(const uint8_t* w, int cb, int nb, int n_rows,
                                               int task, TfPRow<IT, Q6>& r) {
    constexpr int UNITS = 16 / SPR;
    const TfPLane ln = tf_p_lane<SPR>();
    if (task >= (n_rows + UNITS - 1) / UNITS) return;
    const int j = task * UNITS + ln.unit;
    const bool valid = j < n_rows;
    const uint8_t* col = w + (size_t)(valid ? j : 0) * cb;
    if constexpr (Q6) tf_q6k_row_load<SPR, IT>(col, valid, 0, nb, ln.sir, ln.t, r);
    else tf_q4k_row_load<SPR, IT>(col, valid, 0, nb, ln.sir, ln.t, r);
}

// Task `task` of a row GEMV issued unconditionally: a task past the end
// reloads task 0 (its result is dropped), so a ring of such loads keeps exact
// memory waits.
template <int SPR, int IT, bool Q6>
__device__ __forceinline__ void tf_p_rows_load_u(const uint8_t* w, int cb, int nb, int n_rows,
                                                 int task, TfPRow<IT, Q6>& r) {
    constexpr int UNITS = 16 / SPR;
    const TfPLane ln = tf_p_lane<SPR>();
    const int j = task * UNITS + ln.unit;
    const uint8_t* col = w + (size_t)(j < n_rows ? j : 0) * cb;
    if constexpr (Q6) tf_q6k_row_load_u<SPR, IT>(col, nb, ln.sir, ln.t, r);
    else tf_q4k_row_load_u<SPR, IT>(col, nb, ln.sir, ln.t, r);
}

// Ring over this wave's tasks w0, w0 + nwv, ... (nwv waves share the rows):
// r[d] holds task w0 + (k D + d) nwv on entry to round k; every round runs
// all D slots and refills each right after it is consumed, so the memory
// waits stay exact.  EPI as tf_p_rows_run.
template <int SPR, int IT, bool Q6, int D, int EPI, class Res>
__device__ __forceinline__ void tf_p_rows_ring(const uint8_t* w, int cb, int nb, int n_rows,
                                               const TfAct& x, TfPRow<IT, Q6> (&r)[D], int w0,
                                               int nwv, Res res, unsigned long long* fout,
                                               unsigned tag, float* out,
                                               unsigned long long* amax, int slot) {
    constexpr int UNITS = 16 / SPR;
    const TfPLane ln = tf_p_lane<SPR>();
    const int n_tasks = (n_rows + UNITS - 1) / UNITS;
    const bool lead = (ln.lane & (4 * SPR - 1)) == 0;
    unsigned long long best = 0;
    for (int base = w0; base < n_tasks; base += D * nwv) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int task = base + d * nwv;
            const int j = task * UNITS + ln.unit;
            const bool valid = task < n_tasks && j < n_rows;
            float acc;
            if constexpr (Q6) acc = tf_q6k_row_partial<SPR, IT>(r[d], true, 0, nb, ln.sir, ln.t, x);
            else acc = tf_q4k_row_partial<SPR, IT>(r[d], true, 0, nb, ln.sir, ln.t, x);
            const int nt = task + D * nwv;
            tf_p_rows_load_u<SPR, IT, Q6>(w, cb, nb, n_rows, nt < n_tasks ? nt : 0, r[d]);
            acc = tf_group_sum<4 * SPR>(acc);
            if (valid && lead) {
                if constexpr (EPI == 0) {
                    tf_p_putf(fout + j, acc + res(j), tag);
                } else {
                    *(TF_GAS float*)(out + j) = acc;
                    const unsigned long long k = tf_argmax_key(acc, j);
                    best = k > best ? k : best;
                }
            }
        }
    }
    if constexpr (EPI == 1) {
        best = tf_wave_max_u64(best);
        if (ln.lane == 0 && best)
            __hip_atomic_fetch_max((TF_GAS unsigned long long*)amax + (slot % TF_ARGMAX_SLOTS),
                                   best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Rows of one matrix.  EPI 0: residual stream (see below); EPI 1:
// out[j] = dot and the argmax key (lm_head).  The wave's tasks run
// through a ring of D register sets: r[d] holds task wid + (k D + d) nwv,
// and is refilled with the task D steps ahead as soon as it is consumed, so
// D tasks' weights are in flight.  tf_p_rows_prefetch fills the ring (before
// the stage's wait).
template <int SPR, int IT, bool Q6, int D>
__device__ __forceinline__ void tf_p_rows_prefetch(const uint8_t* w, int cb, int nb, int n_rows,
                                                   TfPRow<IT, Q6> (&r)[D]) {
    const int wid = tf_p_wid(), nwv = gridDim.x * TF_P_WAVES;
#pragma unroll
    for (int d = 0; d < D; d++) tf_p_rows_load<SPR, IT, Q6>(w, cb, nb, n_rows, wid + d * nwv, r[d]);
}

// EPI 0 reads the residual from `res` (res(j) -> x_in[j]) and writes
// out[j] = x_in[j] + dot as a flagged word with tag `tag`.
template <int SPR, int IT, bool Q6, int D, int EPI, class Res>
__device__ __forceinline__ void tf_p_rows_run(const uint8_t* w, int cb, int nb, int n_rows,
                                              const TfAct& x, TfPRow<IT, Q6> (&r)[D], Res res,
                                              float res_first,
                                              unsigned long long* fout, unsigned tag,
                                              float* out, unsigned long long* amax) {
    constexpr int UNITS = 16 / SPR;
    const TfPLane ln = tf_p_lane<SPR>();
    const int wid = tf_p_wid(), nwv = gridDim.x * TF_P_WAVES;
    const int n_tasks = (n_rows + UNITS - 1) / UNITS;
    const bool lead = (ln.lane & (4 * SPR - 1)) == 0;
    unsigned long long best = 0;
    for (int base = wid; base < n_tasks; base += D * nwv) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int task = base + d * nwv;
            if (task >= n_tasks) break;  // wave-uniform
            const int j = task * UNITS + ln.unit;
            const bool valid = j < n_rows;
            float acc;
            if constexpr (Q6) acc = tf_q6k_row_partial<SPR, IT>(r[d], valid, 0, nb, ln.sir, ln.t, x);
            else acc = tf_q4k_row_partial<SPR, IT>(r[d], valid, 0, nb, ln.sir, ln.t, x);
            tf_p_rows_load<SPR, IT, Q6>(w, cb, nb, n_rows, task + D * nwv, r[d]);
            acc = tf_group_sum<4 * SPR>(acc);
            if (valid && lead) {
                if constexpr (EPI == 0) {
                    tf_p_putf(fout + j, acc + (task == wid ? res_first : res(j)), tag);
                } else {
                    *(TF_GAS float*)(out + j) = acc;
                    const unsigned long long k = tf_argmax_key(acc, j);
                    best = k > best ? k : best;
                }
            }
        }
    }
    if constexpr (EPI == 1) {
        best = tf_wave_max_u64(best);
        if (ln.lane == 0 && best)
            __hip_atomic_fetch_max((TF_GAS unsigned long long*)amax + (wid % TF_ARGMAX_SLOTS), best,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// --------------------------------------------------- gate/up + SiLU
//
// h = silu(gate x) * up x, published already in Q8 (the activation the down
// projection reads; kernels/gemv.cu:16-65 quantization of the f32 h, so the
// bytes are those tf_quantize_q8 would make of the same h).  Work is dealt
// in half-groups of 16 outputs: workgroup b takes half-groups
// [F/16 b / grid, F/16 (b + 1) / grid), so no workgroup has more than one
// half-group above the fair share; wave w computes outputs 16 h + 2 w, + 1 of
// half-group h in 2 / JPW passes (with SPR <= 8 the even units of a pass take
// gate rows and the odd units the up rows of the same outputs, as
// tf_q4k_pair_rows_kernel; with SPR = 16 a lane loads both rows of one
// output).  A workgroup quantizes each group whose first half it holds: h is
// gathered in LDS and wave 0 quantizes it.  A group split between two
// workgroups has its second half computed first by the later workgroup,
// which publishes those 16 values as tagged f32 words (the exchange area,
// fh + F / 2 + 16 g); the earlier workgroup computes its first half last and
// reads them.  Published group g: words 9 g .. 9 g + 7 hold the 32 Q8 bytes
// (little-endian, 4 per word), word 9 g + 8 the scale d8.

// QKV: waves 1-7 (the compute waves) own the GEMV tasks; every wave polls
// the stage's input, and wave 0, which has no weights in flight (a wave's
// memory counter completes in issue order, so its poll would wait for them
// too), forms the RMS scale.
#define TF_P_CW (TF_P_WAVES - 1)
// Gate/up, whose compute is VALU-bound: every wave prefetches, polls and
// computes a share of the tasks, so each SIMD carries two waves' tasks (with
// seven compute waves one SIMD had one and the other three two); wave 0 also
// quantizes h.  The prefetch the polls wait for comes mostly from the L2 the
// warm-up filled.
// Gate/up tasks in flight per wave: 3 at SPR <= 8; 2 at SPR = 16 (7B widths,
// where the rows are not warmed into the L2 and a deeper prefetch holds up
// the x' poll: 2 / 3 / 4 / 5 gave 511 / 509 / 493 / 491 tok/s on config 4).
#ifndef TF_P_GU_D16
#define TF_P_GU_D16 2
#endif
#ifndef TF_P_GU_D
#define TF_P_GU_D 3
#endif

template <int IT>
struct TfPGuRegs {
    TfQ4kRow<IT> a, b;
};

template <int SPR>
struct TfPGuMap {
    static constexpr int JPW = SPR <= 8 ? 16 / SPR / 2 : 1;  // outputs per task
    static constexpr int HMAX = SPR <= 8 ? 3 : 5;            // half-groups per workgroup
    // tasks per compute wave, and register sets in flight
    static constexpr int K = (16 * HMAX + TF_P_WAVES * JPW - 1) / (TF_P_WAVES * JPW);
    static constexpr int D = SPR <= 8 ? TF_P_GU_D : TF_P_GU_D16;
    static_assert(JPW >= 1 && JPW <= 2, "gate/up lane map needs SPR >= 4");
};

// LDS gather of h: the outputs of the workgroup's half-groups, then (one more
// half-group) the second half of a split group.
__shared__ __align__(16) float tf_p_hbuf[6 * 16];

// Half-groups [s, e) of this workgroup.
struct TfPGuSpan {
    int s, e;
};

__device__ __forceinline__ TfPGuSpan tf_p_gu_span(TfPA& a) {
    const int nh = a.F / 16, b = blockIdx.x, G = gridDim.x;
    return {(int)((long long)nh * b / G), (int)((long long)nh * (b + 1) / G)};
}

// Output (index into the workgroup's outputs, 16 s + o is the row) of task q
// of wave cw, for this lane's unit.
template <int SPR>
__device__ __forceinline__ int tf_p_gu_out(int cw, int q, int unit) {
    const int u = cw + TF_P_WAVES * q;
    if constexpr (SPR <= 8) return u * TfPGuMap<SPR>::JPW + (unit >> 1);
    else return u;
}

// Weights of task q (unconditional; an output past the span loads row j0).
template <int SPR, int IT>
__device__ __forceinline__ void tf_p_gu_load(TfPA& a, TfPL& L, int n_out, int j0, int q,
                                             TfPGuRegs<IT>& r) {
    const TfPLane ln = tf_p_lane<SPR>();
    const int nb = a.E / 256;
    const int o = tf_p_gu_out<SPR>(tf_p_tid() >> 6, q, ln.unit);
    const int j = j0 + (o < n_out ? o : 0);
    if constexpr (SPR <= 8) {
        const uint8_t* w = (ln.unit & 1) ? L.up : L.gate;
        tf_q4k_row_load_u<SPR, IT>(w + (size_t)j * L.cb_gu, nb, ln.sir, ln.t, r.a);
    } else {
        tf_q4k_row_load_u<SPR, IT>(L.gate + (size_t)j * L.cb_gu, nb, ln.sir, ln.t, r.a);
        tf_q4k_row_load_u<SPR, IT>(L.up + (size_t)j * L.cb_gu, nb, ln.sir, ln.t, r.b);
    }
}

// Publishes the Q8 of one 32-value group held as two values per lane of a
// 16-lane row (tf_q8_pair layout, the quantization of tf_quantize_q8) in the
// 9-word group layout: group G_ at words 9 G_ ... ; m = lane & 15.
__device__ __forceinline__ void tf_p_put_pair16_if(unsigned long long* dst, int G_, int m,
                                                   float v0, float v1, unsigned tag, bool put,
                                                   const TfPQ8Rec& rec) {
    const TfQ8Pair r = tf_q8_pair<false>(v0, v1);
    const uint32_t h16 = (uint32_t)(r.q0 & 0xff) | ((uint32_t)(r.q1 & 0xff) << 8);
    const uint32_t other = (uint32_t)tf_dppi<TF_DPP_QUAD_1032>((int)h16);  // lane m ^ 1
    if (put && (m & 1) == 0) tf_p_put(dst + 9 * G_ + (m >> 1), h16 | (other << 16), tag);
    if (put && m == 0) tf_p_put(dst + 9 * G_ + 8, __float_as_uint(r.d), tag);
    if (rec.x && put) {  // the Q8 record
        *reinterpret_cast<float2*>(rec.x + 32 * G_ + 2 * m) = make_float2(v0, v1);
        *reinterpret_cast<uint16_t*>(rec.q + 32 * G_ + 2 * m) = (uint16_t)h16;
        if (m == 0) rec.d[G_] = r.d;
    }
}
__device__ __forceinline__ void tf_p_put_pair16(unsigned long long* dst, int G_, int m, float v0,
                                                float v1, unsigned tag, const TfPQ8Rec& rec) {
    tf_p_put_pair16_if(dst, G_, m, v0, v1, tag, true, rec);
}

// Gate/up tasks of this wave: h = silu(gate) * up of the wave's outputs
// into tf_p_hbuf (and, for the first half-group when it is the second half
// of a group, into the exchange area).  r holds tasks 0 .. D - 1 on entry.
template <int SPR, int IT>
__device__ __forceinline__ void tf_p_gu_compute(TfPA& a, TfPL& L, const TfAct& x,
                                                TfPGuRegs<IT> (&r)[TfPGuMap<SPR>::D],
                                                const TfPGuSpan& sp, unsigned long long* fx,
                                                unsigned tag_x) {
    using M = TfPGuMap<SPR>;
    const TfPLane ln = tf_p_lane<SPR>();
    const int nb = a.E / 256;
    const int cw = tf_p_tid() >> 6;
    const int n_out = 16 * (sp.e - sp.s);
    const int j0 = 16 * sp.s < a.F ? 16 * sp.s : 0;
    const bool sends = (sp.s & 1) && n_out > 0;  // half-group s is a second half
#pragma unroll
    for (int q = 0; q < M::K; q++) {
        TfPGuRegs<IT>& rq = r[q % M::D];
        const int o = tf_p_gu_out<SPR>(cw, q, ln.unit);
        float hv;
        bool writer;
        if constexpr (SPR <= 8) {
            float acc = tf_q4k_row_partial<SPR, IT>(rq.a, true, 0, nb, ln.sir, ln.t, x);
            if (q + M::D < M::K) tf_p_gu_load<SPR, IT>(a, L, n_out, j0, q + M::D, rq);
            acc = tf_group_sum<4 * SPR>(acc);
            const float other = __shfl(acc, (ln.lane + 4 * SPR) & 63, 64);
            hv = (acc / (1.f + __expf(-acc))) * other;
            writer = (ln.unit & 1) == 0 && (ln.lane & (4 * SPR - 1)) == 0;
        } else {
            float g = tf_q4k_row_partial<SPR, IT>(rq.a, true, 0, nb, ln.sir, ln.t, x);
            float u = tf_q4k_row_partial<SPR, IT>(rq.b, true, 0, nb, ln.sir, ln.t, x);
            if (q + M::D < M::K) tf_p_gu_load<SPR, IT>(a, L, n_out, j0, q + M::D, rq);
            g = tf_group_sum<64>(g);
            u = tf_group_sum<64>(u);
            hv = (g / (1.f + __expf(-g))) * u;
            writer = ln.lane == 0;
        }
        if (writer && o < n_out) {
            tf_p_hbuf[o] = hv;
            if (sends && o < 16) tf_p_putf(fx + 16 * (sp.s >> 1) + o, hv, tag_x);
        }
    }
}

// Wave 0 of gate/up, after the compute: reads the second half of a group
// whose first half ends this workgroup's span, then (after the workgroup
// barrier) quantizes the groups whose first half it holds.  False: aborted.
__device__ __forceinline__ void tf_p_gu_exchange(TfPA& a, const TfPGuSpan& sp,
                                                 const unsigned long long* fx, unsigned tag_x) {
    const int lane = tf_p_tid() & 63, last = sp.e - 1;
    if (sp.e <= sp.s || (last & 1)) return;
    const unsigned long long* src = fx + 16 * (last >> 1) + (lane & 15);
    unsigned long long w = tf_ldc64(src);
    for (int spins = 0;;) {
        if (!__builtin_amdgcn_ballot_w64((unsigned)(w >> 32) != tag_x)) break;
        if (++spins > TF_SPIN_LIMIT || ((spins & 15) == 0 && tf_ldu(a.bar + TF_BAR_ABORT))) {
            tf_p_abort(a);
            tf_p_flag = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
        w = tf_ldc64(src);
    }
    if (lane < 16) tf_p_hbuf[16 * (sp.e - sp.s) + lane] = __uint_as_float((unsigned)w);
}

// A workgroup holds at most two such groups (HMAX <= 5 half-groups, the
// first of them possibly the second half of a group): 16-lane row k of the
// wave takes group g0 + k, two values per lane (tf_q8_pair: the same Q8 as
// tf_quantize_q8), so the quantization is a few dozen instructions.
__device__ __forceinline__ void tf_p_gu_quantize(const TfPGuSpan& sp, unsigned long long* fh,
                                                 unsigned tag, const TfPQ8Rec& rec) {
    const int lane = tf_p_tid() & 63;
    const int g0 = (sp.s + 1) >> 1, ng = ((sp.e + 1) >> 1) - g0;
    const int k = lane >> 4, m = lane & 15;  // row k: group g0 + k, values 2 m, 2 m + 1
    const int o = k < ng ? 16 * (2 * (g0 + k) - sp.s) + 2 * m : 0;
    const float2 v = *reinterpret_cast<const float2*>(tf_p_hbuf + o);
    tf_p_put_pair16_if(fh, g0 + k, m, v.x, v.y, tag, k < ng, rec);
}

// Polls a Q8 vector published as 9-word groups (tf_p_put_pair16 layout) into the
// LDS image of nb super-blocks, then forms the per-16 sums (s16) and
// d8 * sum32 (ds) exactly as tf_stage_act does for a Q8 source.
template <int K>
__device__ __forceinline__ bool tf_p_poll_q8img(TfPA& a, uint8_t* lds, int nb,
                                                const unsigned long long* src, unsigned tag) {
    uint32_t* q8w = reinterpret_cast<uint32_t*>(lds);
    float* d8s = reinterpret_cast<float*>(lds + TF_Q8_LDS_BYTES(nb));
    float* dss = d8s + nb * 8;
    int32_t* s16 = reinterpret_cast<int32_t*>(dss + nb * 8);
    const int ng = nb * 8;
    if (!tf_p_poll<K, 1>(
            [&](int i, uint32_t b) {
                const int g = i / 9, w = i - 9 * g;
                if (w < 8) q8w[(tf_q8_pad(32 * g) >> 2) + w] = b;
                else d8s[g] = __uint_as_float(b);
            },
            src, 9 * ng, tag, tf_p_tid(), TF_P_THREADS, a))
        return false;
    for (int g = tf_p_tid(); g < ng; g += TF_P_THREADS) {
        const uint32_t* gw = q8w + (tf_q8_pad(32 * g) >> 2);
        const tf_u32x4 u0 = *reinterpret_cast<const tf_u32x4*>(gw);
        const tf_u32x4 u1 = *reinterpret_cast<const tf_u32x4*>(gw + 4);
        const int one = 0x01010101;
        int sa = tf_dot4(one, (int)u0.x, 0);
        sa = tf_dot4(one, (int)u0.y, sa);
        sa = tf_dot4(one, (int)u0.z, sa);
        sa = tf_dot4(one, (int)u0.w, sa);
        int sb = tf_dot4(one, (int)u1.x, 0);
        sb = tf_dot4(one, (int)u1.y, sb);
        sb = tf_dot4(one, (int)u1.z, sb);
        sb = tf_dot4(one, (int)u1.w, sb);
        s16[2 * g] = sa;
        s16[2 * g + 1] = sb;
        dss[g] = d8s[g] * (float)(sa + sb);
    }
    __syncthreads();
    return true;
}

// ------------------------------------------------------------ attention
//
// Split-KV flash decode (attn/flash.cu:16-255 semantics: per split the
// running max m, normalizer l and unnormalized output O; splits merged with
// the log-sum-exp formula).  A workgroup serves one (kv head, split) pair,
// the split being a run of 64-token tiles; wave g owns query head g of the
// kv head (G = n_head / n_kv <= 8).  Per tile: the workgroup stages K and V
// in LDS (the next tile is already in registers); lane = token for the
// scores (four independent 32-term chains over the head dimension); online
// softmax per wave; lane = two output dims for PV (four independent chains
// over the tokens).  With one split per kv head the wave writes its head's
// output; otherwise it publishes (m, l, O) as tagged words and the first
// workgroup of the kv head polls every split's partial and merges them.

#define TF_P_KROW (TF_P_HD + 8)  // halves per padded K row in LDS

struct TfPAttnLayout {
    static constexpr int K_BYTES = TF_P_TILE * TF_P_KROW * 2;
    static constexpr int V_BYTES = TF_P_TILE * TF_P_HD * 2;
    static constexpr int Q_BYTES = 8 * TF_P_HD * 4;
    static constexpr int P_BYTES = 8 * TF_P_TILE * 4;
    // the waves of a head combine their token slices: per wave (m, l) and O
    static constexpr int C_BYTES = TF_P_WAVES * (2 + TF_P_HD) * 4;
    static constexpr int BYTES = K_BYTES + V_BYTES + Q_BYTES + P_BYTES + C_BYTES;
    static constexpr int CHUNKS = TF_P_TILE * TF_P_HD / 8 / TF_P_THREADS;  // 16 B per thread
};

// A workgroup serves (kv head kh, head group hg, split ws): the split's tiles
// for HPW of the kv head's G query heads.  Each head gets WPH = 8 / HPW waves,
// and wave slice sl takes tokens [sl T, sl T + T) of every 64-token tile
// (T = 64 / WPH).  More head groups spread a short context over more CUs at
// no extra merge cost (the partials stay per head and split); a long context
// keeps one group so each K/V byte is read once.
struct TfPAttnGeo {
    int n_ws, tpw, kh, ws, hg, n_hg, hpw, wph, t_begin, t_end;
    bool active;
};

template <bool MM>
__device__ __forceinline__ TfPAttnGeo tf_p_attn_geo(TfPA& a, int pos) {
    TfPAttnGeo g;
    const int seq = pos + 1;
    const int G = a.H / a.KV;
    const int n_tiles = (seq + TF_P_TILE - 1) / TF_P_TILE;
    const int grid = (int)gridDim.x;
    // the most head groups (4, 2, 1) that still give every tile its own split
    g.n_hg = 1;
    if (G >= 4 && a.KV * n_tiles * 4 <= grid) g.n_hg = 4;
    else if (G >= 2 && a.KV * n_tiles * 2 <= grid) g.n_hg = 2;
    g.hpw = (G + g.n_hg - 1) / g.n_hg;
    g.hpw = g.hpw <= 2 ? 2 : (g.hpw <= 4 ? 4 : 8);  // a power of two dividing 8
    g.n_hg = (G + g.hpw - 1) / g.hpw;
    g.wph = TF_P_WAVES / g.hpw;
    int per_kv = grid / (a.KV * g.n_hg);
    per_kv = per_kv < 1 ? 1 : (per_kv > TF_P_MAX_SPLIT ? TF_P_MAX_SPLIT : per_kv);
    // split length in tokens: whole 64-token tiles, except on the matrix-core
    // path (one head group with one wave per head), whose waves copy 16-token
    // tiles: there 16-token units spread the context over up to per_kv
    // workgroups of a kv head
    const int unit = MM && g.n_hg == 1 && g.wph == 1 ? 16 : TF_P_TILE;
    const int n_units = (seq + unit - 1) / unit;
    const int n0 = n_units < per_kv ? n_units : per_kv;
    const int upw = (n_units + n0 - 1) / n0;
    g.n_ws = (n_units + upw - 1) / upw;  // every split holds at least one unit
    g.tpw = (upw * unit + TF_P_TILE - 1) / TF_P_TILE;
    const int b = blockIdx.x;
    g.active = b < a.KV * g.n_hg * g.n_ws;
    const int kg = g.active ? b / g.n_ws : 0;
    g.kh = kg / g.n_hg;
    g.hg = kg % g.n_hg;
    g.ws = g.active ? b % g.n_ws : 0;
    g.t_begin = g.ws * upw * unit;
    const int te = (g.ws + 1) * upw * unit;
    g.t_end = te < seq ? te : seq;
    return g;
}

struct TfPAttnRegs {
    tf_u32x4 kr[TfPAttnLayout::CHUNKS], vr[TfPAttnLayout::CHUNKS];
};

// Tile t0 -> registers (chunk c = tid + THREADS i: row c / 16, 8 halves at
// 8 (c % 16)).  Unconditional loads from a valid row (see tf_p_poll); rows
// past the split and the row `pos`, produced in this launch, are replaced
// when the tile is stored.
__device__ __forceinline__ void tf_p_attn_load(TfPL& L, int stride, int kh, int t0, int t_end,
                                               int pos, TfPAttnRegs& r) {
    const int tid = tf_p_tid();
    const uint16_t* kb = L.k_cache + (size_t)kh * TF_P_HD;
    const uint16_t* vb = L.v_cache + (size_t)kh * TF_P_HD;
#pragma unroll
    for (int i = 0; i < TfPAttnLayout::CHUNKS; i++) {
        const int c = tid + TF_P_THREADS * i;
        const int row = c / (TF_P_HD / 8), col = 8 * (c % (TF_P_HD / 8));
        const int t = t0 + row;
        const size_t off = (size_t)(t < t_end && t != pos ? t : 0) * stride + col;
        r.kr[i] = tf_ld16(kb + off);
        r.vr[i] = tf_ld16(vb + off);
    }
}

// Static LDS for the new K/V row of this workgroup's kv head (f16 bits).
__shared__ __align__(16) uint16_t tf_p_knew[TF_P_HD], tf_p_vnew[TF_P_HD];

// Partial of (kv head kh, head g, split s): 2 + HD tagged words.
__device__ __forceinline__ unsigned long long* tf_p_part(TfPA& a, int kh, int g, int s) {
    const int G = a.H / a.KV;
    return a.fpart + ((size_t)(kh * G + g) * TF_P_MAX_SPLIT + s) * (2 + TF_P_HD);
}

// Long contexts (one head group: all G <= 8 query heads of the kv head in
// one workgroup) run the split as tf_flash_partial_dma_kernel does: each of
// the 8 waves owns the 16-token tiles j = wave, wave + 8, ... of the split
// and copies them HBM -> LDS itself (global_load_lds_dwordx4) into a private
// two-slot ring, one tile computing while the next is in flight; the first
// two tiles are issued before the q poll.  Per tile, on
// v_mfma_f32_16x16x32_f16 with the query heads padded to 16 (lane l, n =
// l % 16, g = l / 16): S^T[token][head] = K Q^T (q in two f16 parts after
// a power-of-two scale, K f16), the online softmax of head n from a lane max
// and two xor-shuffles, O^T[dim][head] += V^T P^T with p's hi and lo parts
// in one k = 32 step.  The row `pos`, produced in this launch, is patched
// into its LDS slot from the polled K/V row once the slot has landed.  The
// eight waves' (m, l, O) are then combined through LDS and wave h takes
// head h's values in the vector-ALU lane layout, so publication and the
// split merge are unchanged.  LDS rows: a K row's 16-byte chunk c sits at
// chunk c ^ (row % 16); V rows go in blocks of four with 32 bytes of
// padding (both read patterns bank-conflict free).
struct TfPDmaLayout {
    static constexpr int VBLK = 1056;                  // 4 V rows + 32 bytes
    static constexpr int SLOT = 4096 + 4 * VBLK;       // 16 K rows + 16 V rows
    static constexpr int WAVE = 2 * SLOT;              // two-slot ring of a wave
    static constexpr int Q = TF_P_WAVES * WAVE;        // q [G][HD] f32
    static constexpr int BYTES = Q + 16 * TF_P_HD * 4;
    static constexpr int CR = 2 + TF_P_HD + 2;         // combine row: m, l, pad, O
    static constexpr int OL = 69632;                   // merged (O [8][HD], (m, l) [8])
    static_assert(TF_P_WAVES * 16 * CR * 4 <= OL, "combine area");
    static_assert(OL + (8 * TF_P_HD + 16) * 4 <= Q, "merged area");
};
typedef float tf_p_f32x4 __attribute__((ext_vector_type(4)));

// 16-token tile j of the split -> slot b of this wave's ring: four copies of
// 4 K rows, then four of 4 V rows; rows past the split repeat its last token
// (their scores are masked and their V values zeroed when the tile is used).
__device__ __forceinline__ void tf_p_attn_dma_tile(TfPL& L, const TfPAttnGeo& g, int stride,
                                                   uint8_t* lds, int j, int b) {
    const int lane = tf_p_tid() & 63, wave = tf_p_tid() >> 6;
    const int n = lane & 15, r4 = lane >> 4;
    const uint16_t* kb = L.k_cache + (size_t)g.kh * TF_P_HD;
    const uint16_t* vb = L.v_cache + (size_t)g.kh * TF_P_HD;
    const int t0 = g.t_begin + 16 * j;
    const uint32_t base = tf_lds_off(lds) + wave * TfPDmaLayout::WAVE + b * TfPDmaLayout::SLOT;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 4 * i + r4;
        const int t = min(t0 + r, g.t_end - 1);
        tf_lds_dma16(kb + (size_t)t * stride + 8 * (n ^ r), base + 1024 * i);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = min(t0 + 4 * i + r4, g.t_end - 1);
        tf_lds_dma16(vb + (size_t)t * stride + 8 * n, base + 4096 + TfPDmaLayout::VBLK * i);
    }
}

// The wave's first two tiles (before the q poll).
__device__ __forceinline__ void tf_p_attn_dma_prime(TfPL& L, const TfPAttnGeo& g, int stride,
                                                    uint8_t* lds) {
    const int wave = tf_p_tid() >> 6;
    const int n16 = (g.t_end - g.t_begin + 15) / 16;
    if (wave < n16) tf_p_attn_dma_tile(L, g, stride, lds, wave, 0);
    if (wave + TF_P_WAVES < n16) tf_p_attn_dma_tile(L, g, stride, lds, wave + TF_P_WAVES, 1);
}

// Short splits (one 64-token tile, four waves per head: wph = 4, wave w
// scoring the 16 tokens of slice w % 4): waves 0-3 copy slice w HBM -> LDS
// into slot w (the layout of tf_p_attn_dma_tile) before the stage's barrier,
// above the QKV stage's activation image, and the q poll's closing barrier
// publishes the slots; the tile then needs neither register staging nor
// barriers of its own.  Offsets relative to tf_p_dt_base.
struct TfPDtLayout {
    static constexpr int SLOT = TfPDmaLayout::SLOT;
    static constexpr int Q = 4 * SLOT;                    // q [8][HD] f32
    static constexpr int P = Q + 8 * TF_P_HD * 4;         // p [8][TILE]
    static constexpr int C = P + 8 * TF_P_TILE * 4;       // slice combine
    static constexpr int BYTES = C + TF_P_WAVES * (2 + TF_P_HD) * 4;
};
__host__ __device__ __forceinline__ int tf_p_dt_base(int E) {
    return (tf_act_lds_bytes(E / 256, true) + 4 * E + 1023) & ~1023;
}
__device__ __forceinline__ bool tf_p_attn_dt(const TfPAttnGeo& g) {
    return g.tpw == 1 && g.wph == 4;
}
// Slice rows past the split load its last row, and the row `pos` (produced
// in this launch) is read from the polled K/V row instead of its slot.
__device__ __forceinline__ void tf_p_attn_dt_issue(TfPL& L, const TfPAttnGeo& g, int stride,
                                                   uint8_t* lds) {
    const int lane = tf_p_tid() & 63, wave = tf_p_tid() >> 6;
    const int n = lane & 15, r4 = lane >> 4;
    const uint16_t* kb = L.k_cache + (size_t)g.kh * TF_P_HD;
    const uint16_t* vb = L.v_cache + (size_t)g.kh * TF_P_HD;
    if (wave >= 4) return;
    const int t0 = g.t_begin + 16 * wave;
    const uint32_t base = tf_lds_off(lds) + wave * TfPDtLayout::SLOT;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 4 * i + r4;
        const int t = min(t0 + r, g.t_end - 1);
        tf_lds_dma16(kb + (size_t)t * stride + 8 * (n ^ r), base + 1024 * i);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = min(t0 + 4 * i + r4, g.t_end - 1);
        tf_lds_dma16(vb + (size_t)t * stride + 8 * n, base + 4096 + TfPDmaLayout::VBLK * i);
    }
}

// The split's tiles after the q poll; leaves head hd's (m, l) and O dims
// 2 lane, 2 lane + 1 in m, l, o0, o1 of wave hd (valid).
__device__ __forceinline__ void tf_p_attn_dma_run(TfPA& a, TfPL& L, const TfPAttnGeo& g,
                                                  int pos, int stride, uint8_t* lds,
                                                  const float* q_lds, bool valid, int hd,
                                                  float& m_out, float& l_out, float& o0,
                                                  float& o1) {
    using DL = TfPDmaLayout;
    constexpr int HD = TF_P_HD;
    const int tid = tf_p_tid(), lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, gg = lane >> 4;
    const int G = a.H / a.KV;
    const int n16 = (g.t_end - g.t_begin + 15) / 16;
    uint8_t* ring = lds + wave * DL::WAVE;

    // q of head n, dims 32 gg + 8 jj .. +7 (the dim order of the K reads), in
    // two f16 parts of q 2^-e: the largest |q| of the group lands in
    // [2^14, 2^15), the residual of every element within 2^-25 of it
    tf_h16x8 qa[4][2];
    float sc;
    {
        float qv[4][8];
        float qmax = 0.f;
        const bool hv = n < G;
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int h2 = 0; h2 < 2; h2++) {
                float4 v = hv ? *reinterpret_cast<const float4*>(q_lds + n * HD + 32 * gg + 8 * jj + 4 * h2)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
                qv[jj][4 * h2 + 0] = v.x;
                qv[jj][4 * h2 + 1] = v.y;
                qv[jj][4 * h2 + 2] = v.z;
                qv[jj][4 * h2 + 3] = v.w;
                qmax = fmaxf(qmax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
        qmax = tf_wave_max(qmax);
        const int e = qmax > 0.f ? ilogbf(qmax) - 14 : 0;
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x = ldexpf(qv[jj][i], -e);
                const _Float16 p0 = (_Float16)x;
                qa[jj][0][i] = p0;
                qa[jj][1][i] = (_Float16)(x - (float)p0);
            }
        sc = ldexpf(a.scale, e);
    }
    uint32_t koff[4];
#pragma unroll
    for (int jj = 0; jj < 4; jj++) koff[jj] = n * 256 + 16 * ((4 * gg + jj) ^ n);
    const uint32_t voff = 4096 + gg * DL::VBLK + 2 * n;

    float m = TF_P_NEG_BIG, l = 0.f;  // head n: running max, this lane's share of the sum
    tf_p_f32x4 o[8];                  // O^T of dims 16 db + 4 gg + r, head n
#pragma unroll
    for (int db = 0; db < 8; db++) o[db] = tf_p_f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = 0, j = wave; j < n16; k++, j += TF_P_WAVES) {
        if (j + TF_P_WAVES < n16)
            asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // the next tile stays in flight
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint8_t* slot = ring + (k & 1) * DL::SLOT;
        const int t0 = g.t_begin + 16 * j;
        if (pos >= t0 && pos < t0 + 16) {  // wave-uniform: patch the row produced in this launch
            const int rr = pos - t0;
            if (lane < 16) {
                *reinterpret_cast<tf_u32x4*>(slot + rr * 256 + 16 * (lane ^ rr)) =
                    *reinterpret_cast<const tf_u32x4*>(tf_p_knew + 8 * lane);
                *reinterpret_cast<tf_u32x4*>(slot + 4096 + (rr >> 2) * DL::VBLK + (rr & 3) * 256 +
                                             16 * lane) =
                    *reinterpret_cast<const tf_u32x4*>(tf_p_vnew + 8 * lane);
            }
        }
        // ---- scores of tokens t0 + 4 gg + r, head n
        float sv[4];
        {
            tf_h16x8 kf[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) kf[jj] = *reinterpret_cast<const tf_h16x8*>(slot + koff[jj]);
            tf_p_f32x4 c0 = tf_p_f32x4{0.f, 0.f, 0.f, 0.f}, c1 = c0;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                c0 = tf_mfma_f16_k32(kf[jj], qa[jj][0], c0);
                c1 = tf_mfma_f16_k32(kf[jj], qa[jj][1], c1);
            }
            const tf_p_f32x4 c = c0 + c1;
#pragma unroll
            for (int r = 0; r < 4; r++) sv[r] = t0 + 4 * gg + r < g.t_end ? c[r] * sc : TF_P_NEG_BIG;
        }
        // ---- online softmax of head n
        float tm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        tm = fmaxf(tm, __shfl_xor(tm, 16, 64));
        tm = fmaxf(tm, __shfl_xor(tm, 32, 64));
        const float m_new = fmaxf(m, tm);
        const float alpha = __expf(m - m_new);
        m = m_new;
        tf_h16x8 pb;
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = sv[r] > 0.5f * TF_P_NEG_BIG ? __expf(sv[r] - m_new) : 0.f;
            ps += p;
            const _Float16 h0 = (_Float16)p;
            pb[r] = h0;
            pb[4 + r] = (_Float16)(p - (float)h0);
        }
        l = l * alpha + ps;
        // ---- O^T += V^T P^T (hi and lo parts of p in one k = 32 step).  The
        // V values of rows past the split are zeroed, not only their p: those
        // slot rows repeat the row `pos`, whose cache line this launch is
        // still writing (its old bits may be a NaN, and 0 x NaN is NaN).
        {
            _Float16 vv[8][4];
            const uint8_t* vp = slot + voff;
#pragma unroll
            for (int db = 0; db < 8; db++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const _Float16 v = *reinterpret_cast<const _Float16*>(vp + 256 * i + 32 * db);
                    vv[db][i] = t0 + 4 * gg + i < g.t_end ? v : (_Float16)0.f;
                }
#pragma unroll
            for (int db = 0; db < 8; db++) {
                tf_h16x8 va;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    va[i] = vv[db][i];
                    va[4 + i] = vv[db][i];
                }
                o[db] = tf_mfma_f16_k32(va, pb, o[db] * alpha);
            }
        }
        // the slot is consumed: refill it with tile j + 2 waves
        if (j + 2 * TF_P_WAVES < n16) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            tf_p_attn_dma_tile(L, g, stride, lds, j + 2 * TF_P_WAVES, k & 1);
        }
    }

    // ---- the eight waves' (m, l, O) through LDS, merged per head
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    __syncthreads();  // every wave is done with its ring
    float* cmb = reinterpret_cast<float*>(lds);  // [waves][16 heads][CR]
    float* row = cmb + (wave * 16 + n) * DL::CR;
    if (gg == 0) {
        row[0] = m;
        row[1] = l;
    }
#pragma unroll
    for (int db = 0; db < 8; db++)
        *reinterpret_cast<tf_p_f32x4*>(row + 4 + 16 * db + 4 * gg) = o[db];
    __syncthreads();
    float* ol = reinterpret_cast<float*>(lds + DL::OL);  // O [8][HD], then (m, l) [8][2]
    for (int i = tid; i < G * HD; i += TF_P_THREADS) {
        const int h = i / HD, d = i % HD;
        float mw[TF_P_WAVES], M = TF_P_NEG_BIG;
#pragma unroll
        for (int w = 0; w < TF_P_WAVES; w++) {
            mw[w] = cmb[(w * 16 + h) * DL::CR];
            M = fmaxf(M, mw[w]);
        }
        float O = 0.f, Ls = 0.f;
#pragma unroll
        for (int w = 0; w < TF_P_WAVES; w++) {
            const float e = __expf(mw[w] - M);
            O += e * cmb[(w * 16 + h) * DL::CR + 4 + d];
            Ls += e * cmb[(w * 16 + h) * DL::CR + 1];
        }
        ol[h * HD + d] = O;
        if (d == 0) {
            ol[8 * HD + 2 * h] = M;
            ol[8 * HD + 2 * h + 1] = Ls;
        }
    }
    __syncthreads();
    if (valid) {
        m_out = ol[8 * HD + 2 * hd];
        l_out = ol[8 * HD + 2 * hd + 1];
        o0 = ol[hd * HD + 2 * lane];
        o1 = ol[hd * HD + 2 * lane + 1];
    }
}

// Split merge of the matrix-core path: workgroup ws merges the heads
// h = ws, ws + n_ws, ... < G with all eight waves (attn/flash.cu:222-255).
// Wave w polls the O words of splits w, w + 8, ... (lane = dims 2 lane,
// 2 lane + 1) together with every split's (m, l) (lane s holds split s), so
// a head's merge is one poll round for up to 64 splits instead of one per
// 16 splits; M = max_s m_s, w_s = e^(m_s - M), L = sum_s w_s l_s; each wave
// sums w_s O_s over its splits in split order, and the eight wave sums are
// added in wave order through LDS.
__device__ __forceinline__ bool tf_p_attn_merge_wg(TfPA& a, const TfPAttnGeo& g,
                                                   unsigned long long* fo, unsigned to,
                                                   unsigned tp, const TfPQ8Rec& rec) {
    constexpr int HD = TF_P_HD;
    constexpr size_t PS = 2 + HD;
    constexpr int KM = TF_P_MAX_SPLIT / TF_P_WAVES;  // splits per wave at most
    const int tid = tf_p_tid(), lane = tid & 63, wave = tid >> 6;
    const int G = a.H / a.KV;
    float* red = reinterpret_cast<float*>(tf_p_lds);  // [waves][HD]
    for (int h = g.ws; h < G; h += g.n_ws) {  // workgroup-uniform
        const unsigned long long* pbase = tf_p_part(a, g.kh, h, 0);
        const int sl = lane < g.n_ws ? lane : 0;
        unsigned long long wm, wl, w0[KM], w1[KM];
        auto load = [&]() {
            wm = tf_ldc64(pbase + sl * PS);
            wl = tf_ldc64(pbase + sl * PS + 1);
#pragma unroll
            for (int k = 0; k < KM; k++) {
                const int s = wave + TF_P_WAVES * k;
                const int sp = s < g.n_ws ? s : 0;
                w0[k] = tf_ldc64(pbase + sp * PS + 2 + 2 * lane);
                w1[k] = tf_ldc64(pbase + sp * PS + 3 + 2 * lane);
            }
        };
        load();
        for (int spins = 0;;) {
            bool miss = lane < g.n_ws && ((unsigned)(wm >> 32) != tp || (unsigned)(wl >> 32) != tp);
#pragma unroll
            for (int k = 0; k < KM; k++)
                miss |= wave + TF_P_WAVES * k < g.n_ws &&
                        ((unsigned)(w0[k] >> 32) != tp || (unsigned)(w1[k] >> 32) != tp);
            if (!__builtin_amdgcn_ballot_w64(miss)) break;
            if (++spins > TF_SPIN_LIMIT || ((spins & 15) == 0 && tf_ldu(a.bar + TF_BAR_ABORT))) {
                tf_p_abort(a);
                return true;  // the launch is aborted; outputs are not used
            }
            __builtin_amdgcn_s_sleep(2);
            load();
        }
        const float ms = lane < g.n_ws ? __uint_as_float((unsigned)wm) : TF_P_NEG_BIG;
        const float Mx = tf_wave_max(ms);
        const float ws_ = lane < g.n_ws ? __expf(ms - Mx) : 0.f;
        const float Lt = tf_group_sum<64>(ws_ * __uint_as_float((unsigned)wl));
        float A0 = 0.f, A1 = 0.f;
#pragma unroll
        for (int k = 0; k < KM; k++) {
            const int s = wave + TF_P_WAVES * k;
            if (s < g.n_ws) {  // wave-uniform
                const float w = tf_readlane(ws_, s);
                A0 = fmaf(w, __uint_as_float((unsigned)w0[k]), A0);
                A1 = fmaf(w, __uint_as_float((unsigned)w1[k]), A1);
            }
        }
        red[wave * HD + 2 * lane] = A0;
        red[wave * HD + 2 * lane + 1] = A1;
        __syncthreads();
        if (wave == 0) {
            float B0 = 0.f, B1 = 0.f;
#pragma unroll
            for (int w = 0; w < TF_P_WAVES; w++) {
                B0 += red[w * HD + 2 * lane];
                B1 += red[w * HD + 2 * lane + 1];
            }
            const float den = fmaxf(Lt, 1e-20f);
            const int og = ((g.kh * G + h) * HD + 2 * lane) / 32;
            tf_p_put_pair16(fo, og, lane & 15, B0 / den, B1 / den, to, rec);
        }
        __syncthreads();  // red is reused by the next head
    }
    return true;
}

template <bool MM, bool REC>
__device__ __forceinline__ bool tf_p_attn_run(TfPA& a, TfPL& L, const TfPAttnGeo& g, int pos,
                                              TfPAttnRegs& r, uint8_t* lds,
                                              const unsigned long long* fq,
                                              const unsigned long long* fkv, unsigned tq,
                                              unsigned tkv, unsigned long long* fo,
                                              unsigned to, unsigned tp, int sk) {
    using LA = TfPAttnLayout;
    constexpr int HD = TF_P_HD;
    const int tid = tf_p_tid(), lane = tid & 63, wave = tid >> 6;
    const int G = a.H / a.KV, stride = a.KV * HD;
    const TfPQ8Rec rec = tf_p_q8rec<REC>(a, (sk - 1) / 5, 1);
    // matrix-core tiles copied HBM -> LDS per wave, for a single head group
    // with one wave per head (long contexts)
    const bool mm = MM && g.n_hg == 1 && g.wph == 1;
    const bool dt = !mm && tf_p_attn_dt(g);
    uint16_t* k_lds = reinterpret_cast<uint16_t*>(lds);
    uint16_t* v_lds = reinterpret_cast<uint16_t*>(lds + LA::K_BYTES);
    uint8_t* dtl = lds + tf_p_dt_base(a.E);  // the short-split area
    float* q_lds = reinterpret_cast<float*>(mm   ? lds + TfPDmaLayout::Q
                                            : dt ? dtl + TfPDtLayout::Q
                                                 : lds + LA::K_BYTES + LA::V_BYTES);
    float* p_lds = q_lds + 8 * HD;
    // the first two tiles of this wave go out before the poll: the K/V
    // stream overlaps the wait for q
    if (mm) tf_p_attn_dma_prime(L, g, stride, lds);
    // q of the kv head's G query heads (words 0 .. G HD) and the new K/V row
    // (words G HD .. G HD + 2 HD): both vectors in one poll
    {
        const unsigned long long* qsrc = fq + (size_t)g.kh * G * HD;
        const unsigned long long* kvsrc = fkv + (size_t)g.kh * 2 * HD;
        const int nq = G * HD;
        if (!tf_p_poll<3, 1>(
                [&](int i, uint32_t b) {
                    if (i < nq) q_lds[i] = __uint_as_float(b);
                    else if (i < nq + HD) tf_p_knew[i - nq] = (uint16_t)b;
                    else tf_p_vnew[i - nq - HD] = (uint16_t)b;
                },
                TfPSplitSrc{qsrc, kvsrc, nq, tq, tkv}, nq + 2 * HD, 0u, tid, TF_P_THREADS, a))
            return false;
    }
    tf_p_stamp(a, sk, 1);

    // this wave: head hd (valid if hh < hpw and hd < G), token slice sl
    const int hh = wave / g.wph, sl = wave % g.wph;
    const int hd = g.hg * g.hpw + hh;
    const bool valid = hd < G;                   // wave-uniform
    const int T = TF_P_TILE / g.wph;             // tokens per slice
    const int DS = HD / g.wph;                   // dims per lane for the scores
    const int ti = lane % T, ds = lane / T;      // score lane: token ti, dim slice ds
    float m = TF_P_NEG_BIG, l = 0.f, o0 = 0.f, o1 = 0.f;
    const float scale = a.scale;
    float* cm = reinterpret_cast<float*>(
        dt ? dtl + TfPDtLayout::C
           : lds + LA::K_BYTES + LA::V_BYTES + LA::Q_BYTES + LA::P_BYTES);  // [wave][2 + HD]
    if (mm) tf_p_attn_dma_run(a, L, g, pos, stride, lds, q_lds, valid, hd, m, l, o0, o1);
    if (dt && valid && g.t_begin < g.t_end) {
        // the arithmetic of the tile loop below, operands from the wave's slot
        const uint8_t* slot = dtl + sl * TfPDtLayout::SLOT;
        const int t0 = g.t_begin, ts = t0 + 16 * sl, t = ts + ti;
        const bool tv = t < g.t_end;
        const float* qh = q_lds + hd * HD + 32 * ds;
        float sa[4];
#pragma unroll
        for (int dd = 0; dd < 4; dd++) {
            const tf_u32x4 kw =
                t == pos ? *reinterpret_cast<const tf_u32x4*>(tf_p_knew + 32 * ds + 8 * dd)
                         : *reinterpret_cast<const tf_u32x4*>(slot + 256 * ti +
                                                              16 * ((4 * ds + dd) ^ ti));
            const float4 qa = *reinterpret_cast<const float4*>(qh + 8 * dd);
            const float4 qb = *reinterpret_cast<const float4*>(qh + 8 * dd + 4);
            float acc = 0.f;
            acc += qa.x * tf_h2f(kw.x);
            acc += qa.y * tf_h2f(kw.x >> 16);
            acc += qa.z * tf_h2f(kw.y);
            acc += qa.w * tf_h2f(kw.y >> 16);
            acc += qb.x * tf_h2f(kw.z);
            acc += qb.y * tf_h2f(kw.z >> 16);
            acc += qb.z * tf_h2f(kw.w);
            acc += qb.w * tf_h2f(kw.w >> 16);
            sa[dd] = acc;
        }
        float sd = (sa[0] + sa[1]) + (sa[2] + sa[3]);
        sd += tf_swap16(sd);
        sd += __shfl_xor(sd, 32, 64);
        const float sv = tv ? sd * scale : TF_P_NEG_BIG;
        const float m_new = fmaxf(m, tf_wave_max(sv));
        const float alpha = __expf(m - m_new);
        const float e = tv ? __expf(sv - m_new) : 0.f;
        if (lane < 16) p_lds[wave * TF_P_TILE + ti] = e;
        l = l * alpha + tf_group_sum<64>(lane < 16 ? e : 0.f);
        m = m_new;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int tlen = max(0, min(16, g.t_end - ts));
        const float* pw = p_lds + wave * TF_P_TILE;
        const uint32_t vnew = reinterpret_cast<const uint32_t*>(tf_p_vnew)[lane];
        float c0[4] = {0.f, 0.f, 0.f, 0.f}, c1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < 16; tt += 4) {
            if (tt < tlen) {  // wave-uniform
                const float4 pv = *reinterpret_cast<const float4*>(pw + tt);
                const float pp[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int tok = tt + u;  // rows past the split count as zeros
                    uint32_t vv = *reinterpret_cast<const uint32_t*>(
                        slot + 4096 + TfPDmaLayout::VBLK * (tok >> 2) + 256 * (tok & 3) + 4 * lane);
                    vv = ts + tok == pos ? vnew : vv;
                    vv = tok < tlen ? vv : 0u;
                    c0[u] = fmaf(pp[u], tf_h2f(vv), c0[u]);
                    c1[u] = fmaf(pp[u], tf_h2f(vv >> 16), c1[u]);
                }
            }
        }
        o0 = o0 * alpha + ((c0[0] + c0[1]) + (c0[2] + c0[3]));
        o1 = o1 * alpha + ((c1[0] + c1[1]) + (c1[2] + c1[3]));
    }
    for (int it = 0; it < (mm || dt ? 0 : g.tpw); it++) {
        const int t0 = g.t_begin + it * TF_P_TILE;
        __syncthreads();  // the previous tile is consumed
#pragma unroll
        for (int i = 0; i < LA::CHUNKS; i++) {
            const int c = tid + TF_P_THREADS * i;
            const int row = c / (HD / 8), col = 8 * (c % (HD / 8));
            tf_u32x4 kw = r.kr[i], vw = r.vr[i];
            if (t0 + row == pos) {  // the row produced in this launch
                kw = *reinterpret_cast<const tf_u32x4*>(tf_p_knew + col);
                vw = *reinterpret_cast<const tf_u32x4*>(tf_p_vnew + col);
            } else if (t0 + row >= g.t_end) {
                kw = tf_u32x4{0, 0, 0, 0};
                vw = tf_u32x4{0, 0, 0, 0};
            }
            *reinterpret_cast<tf_u32x4*>(k_lds + row * TF_P_KROW + col) = kw;
            *reinterpret_cast<tf_u32x4*>(v_lds + row * HD + col) = vw;
        }
        if (it + 1 < g.tpw) tf_p_attn_load(L, stride, g.kh, t0 + TF_P_TILE, g.t_end, pos, r);
        __syncthreads();
        if (!valid || t0 >= g.t_end) continue;
        // ---- scores: lane (ti, ds) sums dims ds DS .. + DS of token sl T + ti
        // in four chains; the WPH dim slices are then added across lanes
        const int tok = sl * T + ti;
        const int t = t0 + tok;
        const bool tv = t < g.t_end;
        const uint16_t* krow = k_lds + tok * TF_P_KROW + ds * DS;
        const float* qh = q_lds + hd * HD + ds * DS;
        float sa[4] = {0.f, 0.f, 0.f, 0.f};
        for (int dd = 0; dd < DS / 8; dd++) {
            const tf_u32x4 kw = *reinterpret_cast<const tf_u32x4*>(krow + 8 * dd);
            const float4 qa = *reinterpret_cast<const float4*>(qh + 8 * dd);
            const float4 qb = *reinterpret_cast<const float4*>(qh + 8 * dd + 4);
            float acc = sa[dd & 3];
            acc += qa.x * tf_h2f(kw.x);
            acc += qa.y * tf_h2f(kw.x >> 16);
            acc += qa.z * tf_h2f(kw.y);
            acc += qa.w * tf_h2f(kw.y >> 16);
            acc += qb.x * tf_h2f(kw.z);
            acc += qb.y * tf_h2f(kw.z >> 16);
            acc += qb.z * tf_h2f(kw.w);
            acc += qb.w * tf_h2f(kw.w >> 16);
            sa[dd & 3] = acc;
        }
        float sd = (sa[0] + sa[1]) + (sa[2] + sa[3]);
        if (g.wph == 4) {  // slices ds = lane / 16: add lanes ^ 16, ^ 32
            sd += tf_swap16(sd);
            sd += __shfl_xor(sd, 32, 64);
        } else if (g.wph == 2) {  // slices ds = lane / 32
            sd += __shfl_xor(sd, 32, 64);
        }
        const float sv = tv ? sd * scale : TF_P_NEG_BIG;
        // ---- online softmax over the slice's T tokens (each held by WPH lanes)
        const float m_new = fmaxf(m, tf_wave_max(sv));
        const float alpha = __expf(m - m_new);
        const float e = tv ? __expf(sv - m_new) : 0.f;
        if (lane < T) p_lds[wave * TF_P_TILE + ti] = e;
        l = l * alpha + tf_group_sum<64>(lane < T ? e : 0.f);
        m = m_new;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // ---- PV: lane = dims 2 lane, 2 lane + 1 over the slice's tokens, four chains
        const int tlen = max(0, min(T, g.t_end - t0 - sl * T));
        const uint32_t* vcol = reinterpret_cast<const uint32_t*>(v_lds) + (sl * T) * (HD / 2) + lane;
        const float* pw = p_lds + wave * TF_P_TILE;
        float c0[4] = {0.f, 0.f, 0.f, 0.f}, c1[4] = {0.f, 0.f, 0.f, 0.f};
        for (int tt = 0; tt < tlen; tt += 4) {
            const float4 pv = *reinterpret_cast<const float4*>(pw + tt);
            const float pp[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t vv = vcol[(tt + u) * (HD / 2)];
                c0[u] = fmaf(pp[u], tf_h2f(vv), c0[u]);
                c1[u] = fmaf(pp[u], tf_h2f(vv >> 16), c1[u]);
            }
        }
        o0 = o0 * alpha + ((c0[0] + c0[1]) + (c0[2] + c0[3]));
        o1 = o1 * alpha + ((c1[0] + c1[1]) + (c1[2] + c1[3]));
    }
    // ---- the WPH slices of a head: log-sum-exp merge, in slice order, by slice 0
    if (g.wph > 1) {
        float* cw = cm + wave * (2 + HD);
        if (lane == 0) {
            cw[0] = m;
            cw[1] = l;
        }
        cw[2 + 2 * lane] = o0;
        cw[3 + 2 * lane] = o1;
        __syncthreads();
        if (valid && sl == 0) {
            float M = TF_P_NEG_BIG;
            for (int j = 0; j < g.wph; j++) M = fmaxf(M, cm[(wave + j) * (2 + HD)]);
            float Lt = 0.f, A0 = 0.f, A1 = 0.f;
            for (int j = 0; j < g.wph; j++) {
                const float* cj = cm + (wave + j) * (2 + HD);
                const float w = __expf(cj[0] - M);
                Lt = fmaf(w, cj[1], Lt);
                A0 = fmaf(w, cj[2 + 2 * lane], A0);
                A1 = fmaf(w, cj[3 + 2 * lane], A1);
            }
            m = M;
            l = Lt;
            o0 = A0;
            o1 = A1;
        }
    }
    const bool own = valid && sl == 0;  // wave-uniform: this wave carries head hd
    tf_p_stamp(a, sk, 2);
    // output group of this lane's dims: (head, 32-dim group) in Q8
    const int og = ((g.kh * G + hd) * HD + 2 * lane) / 32;
    if (g.n_ws == 1) {
        if (own) {
            const float den = fmaxf(l, 1e-20f);
            tf_p_put_pair16(fo, og, lane & 15, o0 / den, o1 / den, to, rec);
        }
        return true;
    }
    // ---- publish this split's partial; head h is merged by the wave that
    // carries it in split workgroup h mod n_ws (the merges spread over the
    // splits)
    if (own) {
        unsigned long long* pp = tf_p_part(a, g.kh, hd, g.ws);
        if (lane == 0) {
            tf_p_putf(pp, m, tp);
            tf_p_putf(pp + 1, l, tp);
        }
        tf_p_putf(pp + 2 + 2 * lane, o0, tp);
        tf_p_putf(pp + 3 + 2 * lane, o1, tp);
    }
    if (mm) return tf_p_attn_merge_wg(a, g, fo, to, tp, rec);
    if (!own || hd % g.n_ws != g.ws) return true;
    // lane s holds split s's (m, l); lane = dims 2 lane, 2 lane + 1 for O.
    // M = max_s m_s; w_s = e^(m_s - M); L = sum_s w_s l_s; O = sum_s w_s O_s
    // (attn/flash.cu:222-255), the O sum in split order.  The (m, l) words
    // and the O words of the first 16 splits are polled together.
    const unsigned long long* pbase = tf_p_part(a, g.kh, hd, 0);
    constexpr size_t PS = 2 + HD;
    constexpr int CH = 16;  // splits per O poll
    float A0 = 0.f, A1 = 0.f, Lt = 0.f, ws_ = 0.f;
    for (int s0 = 0; s0 < g.n_ws; s0 += CH) {
        const int sl = lane < g.n_ws ? lane : 0;
        unsigned long long wm = 0, wl = 0, w0[CH], w1[CH];
        auto load = [&]() {
            if (s0 == 0) {  // wave-uniform
                wm = tf_ldc64(pbase + sl * PS);
                wl = tf_ldc64(pbase + sl * PS + 1);
            }
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int sp = s0 + u < g.n_ws ? s0 + u : s0;
                w0[u] = tf_ldc64(pbase + sp * PS + 2 + 2 * lane);
                w1[u] = tf_ldc64(pbase + sp * PS + 3 + 2 * lane);
            }
        };
        load();
        for (int spins = 0;;) {
            bool miss = s0 == 0 && lane < g.n_ws &&
                        ((unsigned)(wm >> 32) != tp || (unsigned)(wl >> 32) != tp);
#pragma unroll
            for (int u = 0; u < CH; u++)
                miss |= s0 + u < g.n_ws &&
                        ((unsigned)(w0[u] >> 32) != tp || (unsigned)(w1[u] >> 32) != tp);
            if (!__builtin_amdgcn_ballot_w64(miss)) break;
            if (++spins > TF_SPIN_LIMIT || ((spins & 15) == 0 && tf_ldu(a.bar + TF_BAR_ABORT))) {
                tf_p_abort(a);
                return true;  // the launch is aborted; outputs are not used
            }
            __builtin_amdgcn_s_sleep(2);
            load();
        }
        if (s0 == 0) {
            const float ms = lane < g.n_ws ? __uint_as_float((unsigned)wm) : TF_P_NEG_BIG;
            const float Mx = tf_wave_max(ms);
            ws_ = lane < g.n_ws ? __expf(ms - Mx) : 0.f;
            Lt = tf_group_sum<64>(ws_ * __uint_as_float((unsigned)wl));
        }
#pragma unroll
        for (int u = 0; u < CH; u++) {
            if (s0 + u < g.n_ws) {  // wave-uniform
                const float w = tf_readlane(ws_, s0 + u);
                A0 = fmaf(w, __uint_as_float((unsigned)w0[u]), A0);
                A1 = fmaf(w, __uint_as_float((unsigned)w1[u]), A1);
            }
        }
    }
    const float den = fmaxf(Lt, 1e-20f);
    tf_p_put_pair16(fo, og, lane & 15, A0 / den, A1 / den, to, rec);
    return true;
}

// ------------------------------------------------------------ stages
//
// Each stage runs as its own (non-inlined) function: its prefetch, its
// activation poll, its staging and its GEMV then share one register
// allocation that nothing else in the kernel adds to.  Every stage first
// issues the loads of its first weight tasks (they do not depend on the
// previous stage), then waits at a workgroup barrier (waves that finished
// the previous stage early must not overwrite the LDS image the others are
// still reading; the barrier waits for LDS traffic only, not for the weight
// loads in flight), then polls its input vector.  A false return means the
// launch was aborted.

__device__ __forceinline__ unsigned long long* tf_p_vec(TfPA& a, int kind, int li) {
    const int nbuf = a.nbuf;
    const int par = nbuf == 2 ? (li & 1) : li;
    switch (kind) {
    case TF_PK_XA: return a.fx + (size_t)par * a.E;
    case TF_PK_XB: return a.fx + (size_t)(nbuf + par) * a.E;
    case TF_PK_Q: return a.fq + (size_t)par * a.H * a.HD;
    case TF_PK_KV: return a.fkv + (size_t)par * 2 * a.KV * a.HD;
    case TF_PK_O: return a.fo + (size_t)par * a.H * a.HD;
    default: return a.fh + (size_t)par * a.F;
    }
}

// Polls a flagged vector into the f32 slot of the LDS activation image.
template <int K, int P = 1>
__device__ __forceinline__ bool tf_p_poll_xf(TfPA& a, float* xf, const unsigned long long* src,
                                             int n, unsigned tag) {
    return tf_p_poll<K, P>([&](int i, uint32_t b) { xf[i] = __uint_as_float(b); }, src, n, tag,
                        tf_p_tid(), TF_P_THREADS, a);
}

// Layer li's norm + QKV + RoPE + K/V append.
template <int SPR, int IT, bool REC>
__device__ __forceinline__ bool tf_p_stage_qkv(TfPA* pa, int li, unsigned tb, int pos, int token) {
    uint8_t* lds = tf_p_lds;
    TfPA& a = *pa;
    TfPL& L = tf_p_layer(a, li);
    const int nbE = a.E / 256, tid = tf_p_tid(), wave = tid >> 6;
    constexpr int NS = SPR <= 8 ? 1 : 2;
    const TfAct xE = tf_act_view(lds, nbE);
    // compute waves 1 .. 7 of every workgroup share the tasks, dealt in the
    // wave order 1, 5, 2, 3, 4, 6, 7: waves w and w + 4 share a SIMD, so with
    // five tasks per workgroup (the 3B widths) the two on one SIMD are the
    // first ones, and the last (the heavier Q6_K x f32 V rows) runs alone
    const int wrank = wave == 5 ? 1 : (wave >= 2 && wave <= 4 ? wave : wave - 1);
    const int cwid = wrank * (int)gridDim.x + (int)blockIdx.x, ncw = gridDim.x * TF_P_CW;
    float nw[NS][4];
    tf_p_norm_wload4<NS>(L.attn_norm, a.E, nw);
    // the first two tasks of the wave are loaded before the poll (a wave has
    // two when the rows outnumber the compute waves, e.g. the 7B widths)
    TfPQkvRegs<SPR, IT> rq0, rq1;
    if (wave != 0) {
        tf_p_qkv_load<SPR, IT>(a, L, cwid, rq0);
        tf_p_qkv_load<SPR, IT>(a, L, cwid + ncw, rq1);
    }
    float* raw = tf_p_raw(lds, nbE);
    tf_p_stamp(a, 5 * li, 0);
    __syncthreads();  // the previous stage's LDS readers are done
    if (li == 0) {
        tf_p_rope_table(a.HD, pos, a.theta);
        const int bb = a.embd_q6k ? 210 : 144;
        const uint8_t* col = a.embd + (size_t)token * a.embd_cb;
        for (int i = tid; i < a.E; i += TF_P_THREADS) {
            const uint8_t* blk = col + (size_t)(i >> 8) * bb;
            raw[i] = a.embd_q6k ? tf_q6k_value(blk, i & 255) : tf_q4k_value(blk, i & 255);
        }
        __syncthreads();
        if (wave == 0) {  // the whole wave forms the sum (cross-lane steps)
            const float sc = tf_p_rms_scale(raw, a.E, a.eps);
            if (tid == 0) tf_p_rms = sc;
        }
    } else if (!tf_p_poll_rms_wg<SPR / 2>(a, raw, tf_p_vec(a, TF_PK_XB, li - 1), a.E,
                                          tf_p_tag(tb, li - 1, TF_PK_XB), a.eps)) {
        return false;
    }
    tf_p_stamp(a, 5 * li, 1);
    __syncthreads();  // raw row and scale in LDS
    if (tf_p_flag) return false;
    tf_p_stage8b<true, true, NS>(lds, nbE, raw, tf_p_rms, nw, tf_p_q8rec<REC>(a, li, 0, blockIdx.x == 0));
    tf_p_stamp(a, 5 * li, 2);
    if (wave == 0) return true;
    const TfPQkvGeo g = tf_p_qkv_geo<SPR>(a);
    unsigned long long* fq = tf_p_vec(a, TF_PK_Q, li);
    unsigned long long* fkv = tf_p_vec(a, TF_PK_KV, li);
    const unsigned tq = tf_p_tag(tb, li, TF_PK_Q), tkv = tf_p_tag(tb, li, TF_PK_KV);
    if (cwid < g.n_tasks) tf_p_qkv_task<SPR, IT>(a, L, cwid, pos, xE, rq0, fq, fkv, tq, tkv);
    if (cwid + ncw < g.n_tasks)
        tf_p_qkv_task<SPR, IT>(a, L, cwid + ncw, pos, xE, rq1, fq, fkv, tq, tkv);
    for (int task = cwid + 2 * ncw; task < g.n_tasks; task += ncw) {
        tf_p_qkv_load<SPR, IT>(a, L, task, rq0);
        tf_p_qkv_task<SPR, IT>(a, L, task, pos, xE, rq0, fq, fkv, tq, tkv);
    }
    tf_p_stamp(a, 5 * li, 3, 64);
    return true;
}

// L2 warm-up of the layer's gate/up weights by the workgroups without
// attention work.  Workgroup b runs on XCD b % 8 (the dispatcher deals the
// persistent grid round-robin over the XCDs), and the 32 workgroups of an XCD
// share its 4 MB L2.  During the attention stage HBM is nearly idle, so the
// XCD's non-attention workgroups copy the gate and up row runs of every
// workgroup of their XCD (about 3.2 MB per XCD at the 3B shape) HBM -> LDS,
// into a scratch KB per wave that nothing reads: the lines stay in the L2,
// and the gate/up stage's weight loads, and the drain of its prefetch ahead of
// the x' poll, then run from L2.  The copies start TF_P_WARM_DELAY x 10 ns
// after the stage starts, once the attention workgroups' q poll is done (its
// round trip slows under the extra traffic; 0.5 / 0.8 / 1.0 / 1.2 / 1.5 /
// 2.0 us gave 1019 / 1028 / 1025 / 1022 / 1007 / 980 tok/s), and each wave
// keeps at most 2 TF_P_WARM copies in flight.  Only when the XCD's share fits
// the L2 with room to spare (gate + up at most 28 MB).  Their own wo poll,
// about 5 us later, finds the copies drained.  Only the first TF_P_WARM_PCT %
// of each workgroup's gate and up runs are warmed: with all of them the L2
// evicted about 2.3 MB per layer before the gate/up stage read it (read twice
// from HBM); 100 / 85 / 70 / 60 / 50 / 40 % gave 1027 / 1031 / 1031 / 1029 /
// 1028 / 1017 tok/s and FETCH_SIZE 1,050,687 / 1,021,159 / 1,013,650 /
// 1,012,876 / 1,012,766 / 1,012,892 KiB per launch (warming the last 85 %
// instead of the first: 1016 tok/s).
#ifndef TF_P_WARM
#define TF_P_WARM 4
#endif
#ifndef TF_P_WARM_DELAY
#define TF_P_WARM_DELAY 80
#endif
#ifndef TF_P_WARM_PCT
#define TF_P_WARM_PCT 70
#endif
// scratch above every activation image; it overlaps the short-split attention
// area, which the warming workgroups (those without attention work) do not use
#define TF_P_WARM_LDS 49152

__device__ __forceinline__ void tf_p_gu_warm(TfPA& a, TfPL& L, int n_active) {
    const size_t cb = L.cb_gu;
    if (2 * (size_t)a.F * cb > ((size_t)28 << 20)) return;
    const int G = gridDim.x, b = blockIdx.x, x = b & 7;
    const int per = (G - x + 7) / 8;                            // workgroups on XCD x
    const int att = n_active > x ? (n_active - x + 7) / 8 : 0;  // of them with attention
    const int idx = (b - x) / 8 - att, nidle = per - att;
    if (idx < 0 || nidle <= 0) return;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < TF_P_WARM_DELAY) __builtin_amdgcn_s_sleep(8);
    const int lane = tf_p_tid() & 63, wave = tf_p_tid() >> 6;
    const uint32_t dump = tf_lds_off(tf_p_lds + TF_P_WARM_LDS + 1024 * wave);
    const int nh = a.F / 16;
    const size_t end = (size_t)a.F * cb - 16;
    int issued = 0;
    for (int jj = idx; jj < per; jj += nidle) {
        // the gate/up span of workgroup x + 8 jj (tf_p_gu_span)
        const int bb = x + 8 * jj;
        const int s0 = (int)((long long)nh * bb / G), e0 = (int)((long long)nh * (bb + 1) / G);
        // the first TF_P_WARM_PCT % of each of its gate and up runs
        const size_t pieces =
            ((size_t)16 * (e0 - s0) * cb + 1023) / 1024 * TF_P_WARM_PCT / 100;
        for (size_t pc = wave; pc < 2 * pieces; pc += TF_P_WAVES) {
            const int m = pc >= pieces ? 1 : 0;
            const size_t off = (size_t)16 * s0 * cb + (pc - m * pieces) * 1024 + 16 * lane;
            tf_lds_dma16((m ? L.up : L.gate) + (off < end ? off : end), dump);
            if ((++issued & 3) == 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(TF_P_WARM) : "memory");
        }
    }
}

template <bool MM, bool REC>
__device__ __forceinline__ bool tf_p_stage_attn(TfPA* pa, int li, unsigned tb, int pos) {
    uint8_t* lds = tf_p_lds;
    TfPA& a = *pa;
    TfPL& L = tf_p_layer(a, li);
    const TfPAttnGeo g = tf_p_attn_geo<MM>(a, pos);
    if (!g.active) {
        if constexpr (!MM) tf_p_gu_warm(a, L, a.KV * g.n_hg * g.n_ws);
        return true;
    }
    TfPAttnRegs ra;
    // (the matrix-core path copies its tiles HBM -> LDS after the barrier)
    if (tf_p_attn_dt(g))
        tf_p_attn_dt_issue(L, g, a.KV * TF_P_HD, lds + tf_p_dt_base(a.E));
    else if (!(MM && g.n_hg == 1 && g.wph == 1))
        tf_p_attn_load(L, a.KV * TF_P_HD, g.kh, g.t_begin, g.t_end, pos, ra);
    tf_p_stamp(a, 5 * li + 1, 0);
    __syncthreads();  // the previous stage's LDS readers are done
    const bool ok = tf_p_attn_run<MM, REC>(
        a, L, g, pos, ra, lds, tf_p_vec(a, TF_PK_Q, li), tf_p_vec(a, TF_PK_KV, li),
        tf_p_tag(tb, li, TF_PK_Q), tf_p_tag(tb, li, TF_PK_KV), tf_p_vec(a, TF_PK_O, li),
        tf_p_tag(tb, li, TF_PK_O), tf_p_tag(tb, li, TF_PK_PART), 5 * li + 1);
    tf_p_stamp(a, 5 * li + 1, 3);
    return ok;
}

// x_in[j] of layer li's residual.
__device__ __forceinline__ float tf_p_res_in(TfPA& a, int li, unsigned tb, int token, int j) {
    if (li == 0) {
        const uint8_t* blk = a.embd + (size_t)token * a.embd_cb +
                             (size_t)(j >> 8) * (a.embd_q6k ? 210 : 144);
        return a.embd_q6k ? tf_q6k_value(blk, j & 255) : tf_q4k_value(blk, j & 255);
    }
    const unsigned long long v = tf_ldc64(tf_p_vec(a, TF_PK_XB, li - 1) + j);
    if ((unsigned)(v >> 32) != tf_p_tag(tb, li - 1, TF_PK_XB)) tf_p_abort(a);  // cannot happen
    return __uint_as_float((unsigned)v);
}

template <int SPR, int IT>
__device__ __forceinline__ bool tf_p_stage_wo(TfPA* pa, int li, unsigned tb, int token) {
    uint8_t* lds = tf_p_lds;
    TfPA& a = *pa;
    TfPL& L = tf_p_layer(a, li);
    const int nbE = a.E / 256;
    const TfAct xE = tf_act_view(lds, nbE);
    TfPRow<IT, false> ro[1];
    tf_p_rows_prefetch<SPR, IT, false, 1>(L.wo, L.cb_o, nbE, a.E, ro);
    // the residual of the wave's first row (polled by the QKV stage already)
    const int j0 = tf_p_wid() * (16 / SPR) + tf_p_lane<SPR>().unit;
    const float res0 = j0 < a.E ? tf_p_res_in(a, li, tb, token, j0) : 0.f;
    tf_p_stamp(a, 5 * li + 2, 0);
    __syncthreads();  // the previous stage's LDS readers are done
    if (!tf_p_poll_q8img<(9 * 4096 / 32 + TF_P_THREADS - 1) / TF_P_THREADS>(
            a, lds, nbE, tf_p_vec(a, TF_PK_O, li), tf_p_tag(tb, li, TF_PK_O)))
        return false;
    tf_p_stamp(a, 5 * li + 2, 1);
    tf_p_stamp(a, 5 * li + 2, 2);
    tf_p_rows_run<SPR, IT, false, 1, 0>(
        L.wo, L.cb_o, nbE, a.E, xE, ro, [&](int j) { return tf_p_res_in(a, li, tb, token, j); },
        res0, tf_p_vec(a, TF_PK_XA, li), tf_p_tag(tb, li, TF_PK_XA), nullptr, nullptr);
    tf_p_stamp(a, 5 * li + 2, 3);
    return true;
}

template <int SPR, int IT, bool REC>
__device__ __forceinline__ bool tf_p_stage_gu(TfPA* pa, int li, unsigned tb) {
    using M = TfPGuMap<SPR>;
    constexpr int NS = SPR <= 8 ? 1 : 2;  // staging steps (E <= 2048 NS)
    uint8_t* lds = tf_p_lds;
    TfPA& a = *pa;
    TfPL& L = tf_p_layer(a, li);
    const int nbE = a.E / 256;
    const TfAct xE = tf_act_view(lds, nbE);
    const int wave = tf_p_tid() >> 6;
    const TfPGuSpan sp = tf_p_gu_span(a);
    unsigned long long* fh = tf_p_vec(a, TF_PK_H, li);
    unsigned long long* fx = fh + a.F / 2;  // the exchange area, 16 words per group
    const unsigned tag_x = tf_p_tag(tb, li, TF_PK_HX);
    float* raw = tf_p_raw(lds, nbE);
    // the norm weights first: waiting for them does not wait for the weights
    float nw[NS][4];
    tf_p_norm_wload4<NS>(L.ffn_norm, a.E, nw);
    const int n_out = 16 * (sp.e - sp.s);
    const int j0 = 16 * sp.s < a.F ? 16 * sp.s : 0;
    TfPGuRegs<IT> rg[M::D];
#pragma unroll
    for (int d = 0; d < M::D; d++) tf_p_gu_load<SPR, IT>(a, L, n_out, j0, d, rg[d]);
    if (wave == 0) tf_p_stamp(a, 5 * li + 3, 0);
    __syncthreads();  // the previous stage's LDS readers are done
    // E <= 256 SPR: SPR / 2 words per thread
    if (!tf_p_poll_rms_wg<SPR / 2>(a, raw, tf_p_vec(a, TF_PK_XA, li), a.E,
                                   tf_p_tag(tb, li, TF_PK_XA), a.eps))
        return false;
    if (wave == 0) tf_p_stamp(a, 5 * li + 3, 1);
    __syncthreads();  // raw row and scale in LDS
    if (tf_p_flag) return false;
    tf_p_stage8b<false, true, NS>(lds, nbE, raw, tf_p_rms, nw, tf_p_q8rec<REC>(a, li, 2, blockIdx.x == 0));
    if (wave == 0) tf_p_stamp(a, 5 * li + 3, 2);
    tf_p_gu_compute<SPR, IT>(a, L, xE, rg, sp, fx, tag_x);
    // wave 0 takes the second half of a group whose first half ends the span
    if (wave == 0) tf_p_gu_exchange(a, sp, fx, tag_x);
    __syncthreads();  // h of every wave in LDS
    if (tf_p_flag) return false;
    if (wave == 0) {
        tf_p_gu_quantize(sp, fh, tf_p_tag(tb, li, TF_PK_H), tf_p_q8rec<REC>(a, li, 3));
        tf_p_stamp(a, 5 * li + 3, 3);
    }
    return true;
}

// Down projection: x_out = x_mid + W_down q8(h).
template <int SPR, int IT, bool Q6>
__device__ __forceinline__ bool tf_p_down_body(TfPA& a, TfPL& L, int li, unsigned tb) {
    uint8_t* lds = tf_p_lds;
    const int nbF = a.F / 256;
    const TfAct xF = tf_act_view(lds, nbF);
    TfPRow<IT, Q6> rd[1];
    tf_p_rows_prefetch<SPR, IT, Q6, 1>(L.down, L.cb_down, nbF, a.E, rd);
    // the residual of the wave's first row (polled by the gate/up stage already)
    const unsigned long long* xm = tf_p_vec(a, TF_PK_XA, li);
    const int j0 = tf_p_wid() * (16 / SPR) + tf_p_lane<SPR>().unit;
    const float res0 = __uint_as_float((unsigned)tf_ldc64(xm + (j0 < a.E ? j0 : 0)));
    tf_p_stamp(a, 5 * li + 4, 0);
    __syncthreads();  // the previous stage's LDS readers are done
    // Q8 h: 9 words per 32 values, one pass (up to 19456 values: nbF <= 76)
    if (!tf_p_poll_q8img<(9 * 19456 / 32 + TF_P_THREADS - 1) / TF_P_THREADS>(
            a, lds, nbF, tf_p_vec(a, TF_PK_H, li), tf_p_tag(tb, li, TF_PK_H)))
        return false;
    tf_p_stamp(a, 5 * li + 4, 1);
    tf_p_stamp(a, 5 * li + 4, 2);  // (no staging: h arrives in Q8)
    tf_p_rows_run<SPR, IT, Q6, 1, 0>(
        L.down, L.cb_down, nbF, a.E, xF, rd,
        [&](int j) { return __uint_as_float((unsigned)tf_ldc64(xm + j)); }, res0,
        tf_p_vec(a, TF_PK_XB, li), tf_p_tag(tb, li, TF_PK_XB), nullptr, nullptr);
    tf_p_stamp(a, 5 * li + 4, 3);
    return true;
}

template <int SPR, int IT>
__device__ __forceinline__ bool tf_p_stage_down(TfPA* pa, int li, unsigned tb) {
    TfPA& a = *pa;
    TfPL& L = tf_p_layer(a, li);
    if (L.down_q6k) return tf_p_down_body<SPR, IT, true>(a, L, li, tb);
    return tf_p_down_body<SPR, IT, false>(a, L, li, tb);
}

// Final norm + lm_head + argmax keys; the last workgroup to finish takes the
// argmax and advances the decode state.
__shared__ unsigned long long tf_p_key[TF_P_WAVES];

template <int SPR, int IT, bool REC>
__device__ __forceinline__ bool tf_p_stage_head(TfPA* pa, unsigned tb, int host_mode, int pos,
                                             unsigned gen) {
    uint8_t* lds = tf_p_lds;
    TfPA& a = *pa;
    const int nbE = a.E / 256, tid = tf_p_tid(), L = a.n_layer;
    const TfAct xE = tf_act_view(lds, nbE);
    constexpr int D = TF_P_HEAD_D, NS = SPR <= 8 ? 1 : 2;
    const int nwv = gridDim.x * TF_P_WAVES, w0 = tf_p_wid();
    const int n_tasks = (a.n_vocab + 16 / SPR - 1) / (16 / SPR);
    float nw[NS][4];
    tf_p_norm_wload4<NS>(a.out_norm, a.E, nw);
    TfPRow<IT, true> rh[D];
#pragma unroll
    for (int d = 0; d < D; d++) {
        const int t = w0 + d * nwv;
        tf_p_rows_load_u<SPR, IT, true>(a.head, a.head_cb, nbE, a.n_vocab, t < n_tasks ? t : 0,
                                        rh[d]);
    }
    float* raw = tf_p_raw(lds, nbE);
    tf_p_stamp(a, 5 * L, 0);
    __syncthreads();  // the previous stage's LDS readers are done
    if (!tf_p_poll_rms_wg<SPR / 2>(a, raw, tf_p_vec(a, TF_PK_XB, L - 1), a.E,
                                   tf_p_tag(tb, L - 1, TF_PK_XB), a.eps))
        return false;
    tf_p_stamp(a, 5 * L, 1);
    __syncthreads();  // raw row and scale in LDS
    if (tf_p_flag) return false;
    tf_p_stage8b<false, true, NS>(lds, nbE, raw, tf_p_rms, nw, tf_p_q8rec<REC>(a, L, 0, blockIdx.x == 0));
    tf_p_stamp(a, 5 * L, 2);
    tf_p_rows_ring<SPR, IT, true, D, 1>(a.head, a.head_cb, nbE, a.n_vocab, xE, rh, w0, nwv,
                                        [](int) { return 0.f; }, nullptr, 0u, a.logits, a.amax,
                                        w0);
    tf_p_stamp(a, 5 * L, 3);
    // ticket: the keys of this workgroup are in before its ticket
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.bar + TF_BAR_DONE, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        tf_p_last = prev == gridDim.x - 1;
    }
    __syncthreads();
    if (!tf_p_last) return true;
    unsigned long long k = 0;
    for (int i = tid; i < TF_ARGMAX_SLOTS; i += TF_P_THREADS) {
        const unsigned long long v = tf_ldc64(a.amax + i);
        k = v > k ? v : k;
        tf_stc64(a.amax + i, 0ull);
    }
    k = tf_wave_max_u64(k);
    if ((tid & 63) == 0) tf_p_key[tid >> 6] = k;
    __syncthreads();
    if (tid == 0) {
        for (int w = 0; w < TF_P_WAVES; w++) k = tf_p_key[w] > k ? tf_p_key[w] : k;
        const int next = tf_argmax_key_index(k);
        if (host_mode) {
            tf_stu(reinterpret_cast<unsigned*>(a.argmax), (unsigned)next);
        } else {
            const int st = (int)tf_ldu(reinterpret_cast<unsigned*>(a.step));
            tf_stu(reinterpret_cast<unsigned*>(a.log + st), (unsigned)next);
            const int nf = tf_gld(a.nforced);
            tf_stu(reinterpret_cast<unsigned*>(a.token),
                   (unsigned)(st + 1 < nf ? tf_gld(a.forced + st + 1) : next));
            tf_stu(reinterpret_cast<unsigned*>(a.pos), (unsigned)(pos + 1));
            tf_stu(reinterpret_cast<unsigned*>(a.step), (unsigned)(st + 1));
        }
        tf_stu(a.bar + TF_BAR_DONE, 0u);
        tf_stu(a.bar + TF_BAR_GEN, gen + 1u);
    }
    return true;
}

// ------------------------------------------------------------ the kernel

template <int SPR_E, int IT_E, int SPR_F, int IT_F, bool MM, bool REC>
__global__ __launch_bounds__(TF_P_THREADS) void tf_decode_persistent_kernel(
    const TfPArgs* args, int host_mode, int token_host, int pos_host) {
    {
        const int tid = tf_p_tid();
        const uint32_t* src = reinterpret_cast<const uint32_t*>(args);
        uint32_t* dst = reinterpret_cast<uint32_t*>(&tf_p_args);
        for (int i = tid; i < (int)(sizeof(TfPArgs) / 4); i += TF_P_THREADS) dst[i] = tf_gld(src + i);
        const int nl = tf_gld(&args->n_layer);
        const uint32_t* lsrc = reinterpret_cast<const uint32_t*>(tf_gld(&args->layers));
        uint32_t* ldst = reinterpret_cast<uint32_t*>(tf_p_layers);
        for (int i = tid; i < nl * (int)(sizeof(TfPLayer) / 4); i += TF_P_THREADS)
            ldst[i] = tf_gld(lsrc + i);
        if (tid == 0) tf_p_flag = 0;
        if (tf_gld(&args->trace))
            for (int i = tid; i < (5 * nl + 1) * 4; i += TF_P_THREADS) tf_p_tstamp[i] = 0;
        __syncthreads();
    }
    TfPA& a = *(TfPA*)&tf_p_args;
    const int pos = host_mode ? pos_host : (int)tf_ldu(reinterpret_cast<unsigned*>(a.pos));
    const int token = host_mode ? token_host : (int)tf_ldu(reinterpret_cast<unsigned*>(a.token));
    const unsigned gen = tf_ldu(a.bar + TF_BAR_GEN);
    const unsigned tb = gen * (unsigned)(8 * a.n_layer + 8);
    __syncthreads();
    for (int li = 0; li < a.n_layer; li++) {
        if (!tf_p_stage_qkv<SPR_E, IT_E, REC>(&a, li, tb, pos, token)) return;
        if (!tf_p_stage_attn<MM, REC>(&a, li, tb, pos)) return;
        if (!tf_p_stage_wo<SPR_E, IT_E>(&a, li, tb, token)) return;
        if (!tf_p_stage_gu<SPR_E, IT_E, REC>(&a, li, tb)) return;
        if (!tf_p_stage_down<SPR_F, IT_F>(&a, li, tb)) return;
    }
    tf_p_stage_head<SPR_E, IT_E, REC>(&a, tb, host_mode, pos, gen);
    tf_p_trace_flush(a);
}

// ------------------------------------------------------------ host side

namespace {

int tf_p_lds(const TfPArgs& a) {
    const int nbE = a.E / 256, nbF = a.F / 256;
    int b = tf_act_lds_bytes(nbE, true) + 4 * a.E;
    const int f = tf_act_lds_bytes(nbF, true);
    if (f > b) b = f;
    const int dt = tf_p_dt_base(a.E) + TfPDtLayout::BYTES;
    const int at = TfPAttnLayout::BYTES > dt ? TfPAttnLayout::BYTES : dt;
    b = at > b ? at : b;
    // the warm-up's scratch (tf_p_gu_warm)
    return TF_P_WARM_LDS + TF_P_WAVES * 1024 > b ? TF_P_WARM_LDS + TF_P_WAVES * 1024 : b;
}

struct TfPLaunch {
    const TfPArgs* dev;
    int host_mode, token, pos;
};

template <int SE, int IE, int SF, int IF, bool MM, bool REC>
int tf_p_launch_t(const TfPArgs& a, const TfPLaunch* l, hipStream_t s, int* grid_out,
                  int* lds_out) {
    auto kern = tf_decode_persistent_kernel<SE, IE, SF, IF, MM, REC>;
    const int lds = MM && tf_p_lds(a) < TfPDmaLayout::BYTES ? TfPDmaLayout::BYTES : tf_p_lds(a);
    // the dynamic LDS limit of this instantiation, raised per device to the
    // largest size a model has needed so far
    static std::mutex attr_mu;
    static int attr_lds[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
    {
        std::lock_guard<std::mutex> lk(attr_mu);
        if (attr_lds[dev] < lds) {
            if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    lds) != hipSuccess)
                return (int)hipErrorInvalidValue;
            attr_lds[dev] = lds;
        }
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)kern, TF_P_THREADS,
                                                     lds) != hipSuccess ||
        per_cu < 1)
        return (int)hipErrorInvalidConfiguration;
    int grid = tf_device_cus();
    if (grid > TF_P_MAX_WG) grid = TF_P_MAX_WG;
    // the gate/up task tables hold TfPGuMap<SE>::HMAX half-groups per workgroup
    if ((a.F / 16 + grid - 1) / grid > TfPGuMap<SE>::HMAX) return (int)hipErrorInvalidValue;
    if (grid_out) *grid_out = grid;
    if (lds_out) *lds_out = lds;
    if (!l) return 0;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(TF_P_THREADS), lds, s, l->dev, l->host_mode,
                       l->token, l->pos);
    return (int)hipGetLastError();
}

// Instantiations: (SPR, ITERS) of the model width and of the FFN width.
// One wave per query head of a kv head (G <= 8); the FFN width also bounds
// the unrolled poll of h (22 words per thread in one pass, or 19 in two).
template <class F>
int tf_p_dispatch(int E, int F_, int H, int KV, int HD, F&& f) {
    if (HD != TF_P_HD || KV <= 0 || H % KV || H / KV > TF_P_WAVES) return -1;
    const int nbE = E / 256, nbF = F_ / 256;
    if (nbE <= 4 && nbF <= 4) return f(std::integral_constant<int, 0>{});
    if (nbE > 4 && nbE <= 8 && nbF > 32 && nbF <= 44) return f(std::integral_constant<int, 1>{});
    if (nbE > 8 && nbE <= 16 && nbF > 64 && nbF <= 76) return f(std::integral_constant<int, 2>{});
    return -1;
}

// MM: the instantiation whose attention runs long contexts on the matrix
// cores (its extra registers would cost the short-context step ~2%).
// REC: the instantiation that keeps the Q8 record (TfPArgs::q8x set).
template <int V, bool MM, bool REC>
int tf_p_call_r(const TfPArgs& a, const TfPLaunch* l, hipStream_t s, int* grid, int* lds) {
    if constexpr (V == 0) return tf_p_launch_t<4, 1, 4, 1, MM, REC>(a, l, s, grid, lds);
    else if constexpr (V == 1) return tf_p_launch_t<8, 1, 16, 3, MM, REC>(a, l, s, grid, lds);
    else return tf_p_launch_t<16, 1, 16, 5, MM, REC>(a, l, s, grid, lds);
}
template <int V, bool MM>
int tf_p_call(const TfPArgs& a, const TfPLaunch* l, hipStream_t s, int* grid, int* lds) {
    return a.q8x ? tf_p_call_r<V, MM, true>(a, l, s, grid, lds)
                 : tf_p_call_r<V, MM, false>(a, l, s, grid, lds);
}

}  // namespace

bool tf_decode_persistent_supported(int n_layer, int E, int F, int H, int KV, int HD) {
    if (n_layer < 1 || n_layer > TF_P_MAX_LAYERS || E % 256 || F % 256 || H * HD != E)
        return false;
    return tf_p_dispatch(E, F, H, KV, HD, [](auto) { return 0; }) == 0;
}

bool tf_decode_persistent_long_ctx(const TfPArgs& a, int grid, int pos) {
    const int G = a.H / a.KV;
    // tf_p_attn_geo: one head group with one wave per head
    const int n_tiles = (pos + 1 + TF_P_TILE - 1) / TF_P_TILE;
    if (G >= 4 && a.KV * n_tiles * 4 <= grid) return false;
    if (G >= 2 && a.KV * n_tiles * 2 <= grid) return false;
    return G > 4;
}

int tf_decode_persistent_grid(const TfPArgs& a, int* lds_bytes) {
    int grid = 0;
    const int rc = tf_p_dispatch(a.E, a.F, a.H, a.KV, a.HD, [&](auto v) {
        return tf_p_call<decltype(v)::value, false>(a, nullptr, nullptr, &grid, lds_bytes);
    });
    return rc == 0 ? grid : 0;
}

int tf_decode_persistent_launch(const TfPArgs& a, const TfPArgs* dev, int host_mode, int token,
                                int pos, hipStream_t stream, bool long_ctx) {
    if (!dev) return (int)hipErrorInvalidValue;
    const TfPLaunch l{dev, host_mode, token, pos};
    const int rc = tf_p_dispatch(a.E, a.F, a.H, a.KV, a.HD, [&](auto v) {
        return long_ctx ? tf_p_call<decltype(v)::value, true>(a, &l, stream, nullptr, nullptr)
                        : tf_p_call<decltype(v)::value, false>(a, &l, stream, nullptr, nullptr);
    });
    return rc < 0 ? (int)hipErrorInvalidValue : rc;
}

// ------------------------------------------------ quantizer check entry
//
// The step's two in-kernel quantizers applied to a plain f32 vector, so that
// their bytes can be compared with tf_quantize_q8 (kernels/gemv.cu:43-65) on
// chosen inputs (near-ties, subnormal scales, zero groups): variant 0 is the
// eight-lane staging of the norm inputs (tf_q8_g8, four values per lane),
// variant 1 the sixteen-lane form of the attention output and of h
// (tf_q8_pair, two values per lane).
__global__ __launch_bounds__(256) void tf_p_q8_check_kernel(const float* __restrict__ x,
                                                             int8_t* __restrict__ q,
                                                             float* __restrict__ d, int n,
                                                             int variant) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (variant == 0) {
        const int e = 4 * t;  // groups never straddle a workgroup (256 x 4 = 32 x 32)
        const bool live = e < n;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = live ? x[e + i] : 0.f;
        const TfQ8Quad r = tf_q8_g8<false>(v);
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; i++) q[e + i] = (int8_t)r.q[i];
            if ((t & 7) == 0) d[e / 32] = r.d;
        }
    } else {
        const int e = 2 * t;
        const bool live = e < n;
        const TfQ8Pair r = tf_q8_pair<false>(live ? x[e] : 0.f, live ? x[e + 1] : 0.f);
        if (live) {
            q[e] = (int8_t)r.q0;
            q[e + 1] = (int8_t)r.q1;
            if ((t & 15) == 0) d[e / 32] = r.d;
        }
    }
}

extern "C" int tf_decode_step_quantize_q8(const float* x, int n, int variant, int8_t* q,
                                          float* d, tf_stream_t stream) {
    TF_CHECK_ARG(x && q && d && n > 0 && n % 32 == 0 && (variant == 0 || variant == 1));
    const int per = variant == 0 ? 4 : 2;  // values per thread
    const int threads = n / per;
    hipLaunchKernelGGL(tf_p_q8_check_kernel, dim3((threads + 255) / 256), dim3(256), 0,
                       tf_stream(stream), x, q, d, n, variant);
    return TF_LAUNCH_RESULT();
}
