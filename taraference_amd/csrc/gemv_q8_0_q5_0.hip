// GEMVs over the 32-value block formats Q8_0 and Q5_0 (batch 1), gfx950.
//
// Replaces kernels/gemv.cu dot_q8_0_col_q8_range + gemv_q8_0_global
// (:1558-1635), gemv_q8_0 (:1585), gemv_q8_0_global_splitk (:1725),
// gemv_q5_0 (:1751), gemv_q8_0_splitk (:2117), gemv_q5_0_splitk (:2158),
// dot_q5_0_col_xs + gemv_q5_0_qk (:2268-2343), gemv_q5_0_qkv (:2710) and
// gemv_q8_0_qkv (:2766).
//
// Formats (per 32 values):
//   Q8_0, 34 B: f16 d | int8 qs[32]                    value t = d * qs[t]
//   Q5_0, 22 B: f16 d | u32 qh | u8 qs[16]             value t = d * (code - 16)
//     code t < 16 = low nibble of qs[t] | bit t of qh << 4,
//     code 16 + t = high nibble of qs[t] | bit 16 + t of qh << 4.
//
// Work split.  A row (output column) is spread over SPR four-lane quads of
// one wave; 16 / SPR rows share a wave and the grid is persistent.
//  * Q8_0 x Q8, fast layout (even block count, dword-aligned columns): a
//    quad owns a PAIR of blocks, 68 bytes = 17 dwords, one 16-byte load per
//    lane plus the shared 17th dword, so a wave streams contiguous memory.
//    The activation is staged in LDS as the same 68-byte pair image with
//    zero bytes where the weights hold d, so each lane's v_dot4 over its
//    dwords is the int8 product of its bytes; the per-block int32 sums are
//    formed exactly (quad DPP) and scaled as dw * xd * sum, the reference's
//    per-block arithmetic.
//  * Q8_0 x Q8, any layout: a quad owns a block; lane p takes qs[8p..8p+7]
//    (16-bit loads, the blocks are only 2-byte aligned).
//  * f32 activations (Q5_0, and the f32 split-K Q8_0): a quad owns a block,
//    fp32 products as the reference; the staged activation is permuted per
//    block so that every lane reads its eight values as two 16-byte LDS
//    reads.
#include <type_traits>

#include "tf_common.hpp"
#include "tf_host.hpp"

enum TfB32Fmt { TF_B32_Q8_PAIR = 0, TF_B32_Q8_GEN = 1, TF_B32_Q8_F32 = 2, TF_B32_Q5_F32 = 3 };
enum TfB32Src { TF_B32_SRC_Q8 = 0, TF_B32_SRC_F32 = 1 };

// Up to three matrices with the same K (Q/K/V or Q/K) share one launch;
// their columns are numbered one after the other.  With n_split >= 1 there
// is one matrix and out[0] receives partial[s * n + j] for block split s.
struct TfB32Job {
    const uint8_t* w[3];
    float* out[3];
    const float* bias[3];
    int n[3];
    int n_tot;  // tasks: n[0]+n[1]+n[2], or n_split * n[0]
    int nb;     // blocks per column
    int col_bytes;
    int n_split;  // 0: whole columns
    int use_res;
    const float* residual;
    const int8_t* xq;  // TF_B32_SRC_Q8
    const float* xd;
    const float* x;  // TF_B32_SRC_F32
};

// ------------------------------------------------------------ LDS images

// Pair image (TF_B32_Q8_PAIR): pair k of groups at 80 k (16-byte aligned):
// bytes 0-1 zero | q8 of group 2k | 2 bytes zero | q8 of group 2k+1 (the
// same byte positions as two Q8_0 blocks), then 12 unused bytes.
__host__ __device__ constexpr int tf_b32_q8_off(int fmt, int g) {
    return fmt == TF_B32_Q8_PAIR ? 80 * (g >> 1) + 2 + 34 * (g & 1) : 32 * g;
}
__host__ __device__ constexpr int tf_b32_q8_bytes(int fmt, int G) {
    return fmt == TF_B32_Q8_PAIR ? 80 * ((G + 1) >> 1) : 32 * G;
}
__host__ __device__ constexpr int tf_b32_lds_bytes(int fmt, int G) {
    return fmt <= TF_B32_Q8_GEN ? tf_b32_q8_bytes(fmt, G) + 4 * G : 128 * G;
}
// f32 image: value 32 g + v at float 32 g + tf_b32_xperm(fmt, v).  Q5_0 lane
// p of a quad reads values 4p..4p+3 and 16+4p..16+4p+3 as floats 8p..8p+7.
__device__ __forceinline__ int tf_b32_xperm(int fmt, int v) {
    if (fmt != TF_B32_Q5_F32) return v;
    return ((v & 15) >> 2) * 8 + (v >> 4) * 4 + (v & 3);
}

// Build the activation image; all threads of the workgroup; ends with a
// barrier.  Quantization (f32 source, Q8 formats) is the reference's
// (kernels/gemv.cu:16-40), bit-identical to tf_quantize_q8: a 16-lane DPP
// row holds one group as value pairs.
template <int FMT, int SK>
__device__ __forceinline__ void tf_b32_stage(const TfB32Job& jb, uint8_t* lds) {
    const int G = jb.nb;
    if constexpr (FMT >= TF_B32_Q8_F32) {
        float* xs = reinterpret_cast<float*>(lds);
        for (int i = threadIdx.x; i < G * 8; i += blockDim.x) {
            const float4 v = *reinterpret_cast<const float4*>(jb.x + 4 * i);
            const int g = i >> 3, v0 = 4 * (i & 7);
            *reinterpret_cast<float4*>(xs + 32 * g + tf_b32_xperm(FMT, v0)) = v;
        }
    } else {
        int8_t* q8 = reinterpret_cast<int8_t*>(lds);
        float* d8 = reinterpret_cast<float*>(lds + tf_b32_q8_bytes(FMT, G));
        if constexpr (SK == TF_B32_SRC_Q8) {
            for (int g = threadIdx.x; g < G; g += blockDim.x) {
                uint16_t* dst = reinterpret_cast<uint16_t*>(q8 + tf_b32_q8_off(FMT, g));
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t v = tf_gld(reinterpret_cast<const uint32_t*>(jb.xq) + 8 * g + i);
                    dst[2 * i] = (uint16_t)v;
                    dst[2 * i + 1] = (uint16_t)(v >> 16);
                }
                if (FMT == TF_B32_Q8_PAIR) dst[-1] = 0;  // the d slot of this block
                d8[g] = tf_gld(jb.xd + g);
            }
        } else {
            const int m = threadIdx.x & 15, rows = blockDim.x >> 4;
            for (int g0 = 0; g0 < G; g0 += rows) {  // workgroup-uniform trip count
                const int g = g0 + (threadIdx.x >> 4);
                const bool ok = g < G;
                const float2 v = ok ? *reinterpret_cast<const float2*>(jb.x + 32 * g + 2 * m)
                                    : make_float2(0.f, 0.f);
                const TfQ8Pair r = tf_q8_pair<false>(v.x, v.y);
                if (ok) {
                    uint16_t* dst = reinterpret_cast<uint16_t*>(q8 + tf_b32_q8_off(FMT, g));
                    dst[m] = (uint16_t)((r.q0 & 0xff) | ((r.q1 & 0xff) << 8));
                    if (m == 0) {
                        d8[g] = r.d;
                        if (FMT == TF_B32_Q8_PAIR) dst[-1] = 0;
                    }
                }
            }
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------ per-row work

__device__ __forceinline__ uint32_t tf_b32_u16(const uint8_t* p) {
    return *(const TF_GAS uint16_t*)p;
}
__device__ __forceinline__ uint32_t tf_b32_u32_a2(const uint8_t* p) {
    return tf_b32_u16(p) | (tf_b32_u16(p + 2) << 16);
}

// Weights of one quad-step of a row, loaded before any of them is used.
struct TfB32Regs {
    tf_u32x4 a;   // PAIR: dwords 4p..4p+3 of the pair; GEN / Q8_F32: qs bytes
                  // 8p..8p+7 in a.x, a.y; Q5: qs bytes 4p..4p+3 in a.x
    uint32_t e;   // PAIR: dword 16; Q5: qh
    uint32_t d;   // GEN / Q8_F32 / Q5: f16 bits of d
};

template <int FMT>
__device__ __forceinline__ void tf_b32_load(const uint8_t* col, int k, int p, TfB32Regs& r) {
    if constexpr (FMT == TF_B32_Q8_PAIR) {
        const uint8_t* base = col + 68 * k;
        r.a = tf_ld16_a4(base + 16 * p);
        r.e = tf_gld(reinterpret_cast<const uint32_t*>(base + 64));
        r.d = 0;
    } else if constexpr (FMT == TF_B32_Q5_F32) {
        const uint8_t* base = col + 22 * k;
        r.d = tf_b32_u16(base);
        r.e = tf_b32_u32_a2(base + 2);
        r.a.x = tf_b32_u32_a2(base + 6 + 4 * p);
    } else {
        const uint8_t* base = col + 34 * k;
        r.d = tf_b32_u16(base);
        r.a.x = tf_b32_u32_a2(base + 2 + 8 * p);
        r.a.y = tf_b32_u32_a2(base + 6 + 8 * p);
    }
}

template <int CTRL>
__device__ __forceinline__ uint32_t tf_dppu(uint32_t v) {
    return (uint32_t)tf_dppi<CTRL>((int)v);
}
#define TF_DPP_QUAD_0000 0x00  // quad_perm [0,0,0,0]
#define TF_DPP_QUAD_2222 0xAA  // quad_perm [2,2,2,2]

// Contribution of one quad-step (unit k: pair k for PAIR, block k otherwise)
// to the row sum; blocks outside [b0, b1) add nothing.  For the Q8 formats
// only lane 0 of the quad returns a non-zero value.
template <int FMT>
__device__ __forceinline__ float tf_b32_step(const TfB32Regs& r, int k, int p, int b0, int b1,
                                             const uint8_t* lds, int G) {
    if constexpr (FMT == TF_B32_Q8_PAIR) {
        const int8_t* q8 = reinterpret_cast<const int8_t*>(lds);
        const float* d8 = reinterpret_cast<const float*>(lds + tf_b32_q8_bytes(FMT, G));
        const tf_u32x4 x = *reinterpret_cast<const tf_u32x4*>(q8 + 80 * k + 16 * p);
        const int xe = p == 3 ? *reinterpret_cast<const int*>(q8 + 80 * k + 64) : 0;
        const int t0 = tf_dot4((int)r.a.x, (int)x.x, 0);
        int rest = tf_dot4((int)r.a.y, (int)x.y, 0);
        rest = tf_dot4((int)r.a.z, (int)x.z, rest);
        rest = tf_dot4((int)r.a.w, (int)x.w, rest);
        const int e = tf_dot4((int)r.e, xe, 0);
        int sa = p < 2 ? t0 + rest : (p == 2 ? t0 : 0);
        int sb = p == 2 ? rest : (p == 3 ? t0 + rest + e : 0);
        sa += tf_dppi<TF_DPP_QUAD_1032>(sa);
        sa += tf_dppi<TF_DPP_QUAD_2301>(sa);
        sb += tf_dppi<TF_DPP_QUAD_1032>(sb);
        sb += tf_dppi<TF_DPP_QUAD_2301>(sb);
        const uint32_t da = tf_dppu<TF_DPP_QUAD_0000>(r.a.x);        // lane 0: bytes 0-1
        const uint32_t db = tf_dppu<TF_DPP_QUAD_2222>(r.a.x) >> 16;  // lane 2: bytes 34-35
        const int A = 2 * k, B = 2 * k + 1;
        float acc = 0.f;
        if (p == 0 && A >= b0 && A < b1) acc += tf_h2f(da) * d8[A] * (float)sa;
        if (p == 0 && B >= b0 && B < b1) acc += tf_h2f(db) * d8[B] * (float)sb;
        return acc;
    } else if constexpr (FMT == TF_B32_Q8_GEN) {
        const int8_t* q8 = reinterpret_cast<const int8_t*>(lds);
        const float* d8 = reinterpret_cast<const float*>(lds + tf_b32_q8_bytes(FMT, G));
        const tf_u32x2 x = *reinterpret_cast<const tf_u32x2*>(q8 + 32 * k + 8 * p);
        int s = tf_dot4((int)r.a.x, (int)x.x, 0);
        s = tf_dot4((int)r.a.y, (int)x.y, s);
        s += tf_dppi<TF_DPP_QUAD_1032>(s);
        s += tf_dppi<TF_DPP_QUAD_2301>(s);
        return (p == 0 && k >= b0 && k < b1) ? tf_h2f(r.d) * d8[k] * (float)s : 0.f;
    } else {
        const float* xs = reinterpret_cast<const float*>(lds) + 32 * k + 8 * p;
        const float4 xa = *reinterpret_cast<const float4*>(xs);
        const float4 xb = *reinterpret_cast<const float4*>(xs + 4);
        float s;
        if constexpr (FMT == TF_B32_Q8_F32) {
            const uint32_t u = r.a.x, v = r.a.y;
            s = (float)(int8_t)u * xa.x;
            s += (float)(int8_t)(u >> 8) * xa.y;
            s += (float)(int8_t)(u >> 16) * xa.z;
            s += (float)(int8_t)(u >> 24) * xa.w;
            s += (float)(int8_t)v * xb.x;
            s += (float)(int8_t)(v >> 8) * xb.y;
            s += (float)(int8_t)(v >> 16) * xb.z;
            s += (float)(int8_t)(v >> 24) * xb.w;
        } else {
            // codes of values 4p+i (low nibbles) and 16+4p+i (high nibbles)
            const uint32_t q = r.a.x, hl = r.e >> (4 * p), hh = r.e >> (16 + 4 * p);
            auto code = [&](int i, bool high) -> float {
                const uint32_t nib = high ? (q >> (8 * i + 4)) & 15u : (q >> (8 * i)) & 15u;
                const uint32_t hb = ((high ? hh : hl) >> i) & 1u;
                return (float)((int)(nib | (hb << 4)) - 16);
            };
            s = code(0, false) * xa.x;
            s += code(1, false) * xa.y;
            s += code(2, false) * xa.z;
            s += code(3, false) * xa.w;
            s += code(0, true) * xb.x;
            s += code(1, true) * xb.y;
            s += code(2, true) * xb.z;
            s += code(3, true) * xb.w;
        }
        return (k >= b0 && k < b1) ? tf_h2f(r.d) * s : 0.f;
    }
}

// Task t -> (column pointer, output slot, block range).
struct TfB32Task {
    const uint8_t* col;
    float* out;
    const float* bias;
    int j;
    int b0, b1;
    bool valid;
};

__device__ __forceinline__ TfB32Task tf_b32_task(const TfB32Job& jb, int t) {
    TfB32Task r;
    r.valid = t < jb.n_tot;
    const int tt = r.valid ? t : 0;
    if (jb.n_split > 0) {
        const int s = tt / jb.n[0], j = tt - s * jb.n[0];
        r.col = jb.w[0] + (size_t)j * jb.col_bytes;
        r.out = jb.out[0] + (size_t)s * jb.n[0];
        r.bias = nullptr;
        r.j = j;
        r.b0 = (jb.nb * s) / jb.n_split;
        r.b1 = (jb.nb * (s + 1)) / jb.n_split;
    } else {
        const int m = tt < jb.n[0] ? 0 : (tt < jb.n[0] + jb.n[1] ? 1 : 2);
        const int j = tt - (m > 0 ? jb.n[0] : 0) - (m > 1 ? jb.n[1] : 0);
        r.col = jb.w[m] + (size_t)j * jb.col_bytes;
        r.out = jb.out[m];
        r.bias = jb.bias[m];
        r.j = j;
        r.b0 = 0;
        r.b1 = jb.nb;
    }
    return r;
}

// ------------------------------------------------------------------ kernel

// SPR quads per row (4, 8 or 16).  ITERS > 0: every quad has at most ITERS
// units of work per row, all loaded up front, and the next task's loads are
// issued before this task is computed; ITERS == 0: a plain loop.
template <int FMT, int SK, int SPR, int ITERS>
__global__ __launch_bounds__(512) void tf_b32_kernel(TfB32Job jb) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int UNITS = 16 / SPR;
    const int lane = threadIdx.x & 63;
    const int p = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
    const int wave = tf_wave_id();
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    const int n_tasks = (jb.n_tot + UNITS - 1) / UNITS;
    const int G = jb.nb;
    constexpr bool PAIR = FMT == TF_B32_Q8_PAIR;
    // work units of a row (pairs for PAIR, blocks otherwise) over [b0, b1)
    auto u_lo = [&](const TfB32Task& t) { return PAIR ? (t.b0 >> 1) : t.b0; };
    auto u_hi = [&](const TfB32Task& t) { return PAIR ? ((t.b1 + 1) >> 1) : t.b1; };

    auto finish = [&](const TfB32Task& t, float acc) {
        acc = tf_group_sum<4 * SPR>(acc);
        if (t.valid && (lane & (4 * SPR - 1)) == 0) {
            if (jb.n_split == 0) {
                if (jb.use_res == 1) acc += jb.residual[t.j];
                else if (jb.use_res == 2) acc += t.out[t.j];
                if (t.bias) acc += t.bias[t.j];
            }
            t.out[t.j] = acc;
        }
    };

    int task = wave;
    if constexpr (ITERS > 0) {
        TfB32Regs cur[ITERS], nxt[ITERS];
        TfB32Task tc = tf_b32_task(jb, task * UNITS + unit);
        auto load_all = [&](const TfB32Task& t, TfB32Regs (&r)[ITERS]) {
            const int lo = u_lo(t), hi = u_hi(t);
#pragma unroll
            for (int i = 0; i < ITERS; i++) {
                const int k = lo + sir + i * SPR;
                tf_b32_load<FMT>(t.col, k < hi ? k : lo, p, r[i]);  // clamped: no branch
            }
        };
        if (task < n_tasks) load_all(tc, cur);
        tf_b32_stage<FMT, SK>(jb, lds);
        for (; task < n_tasks; task += nwaves) {
            const int nt = task + nwaves;
            const TfB32Task tn = tf_b32_task(jb, nt * UNITS + unit);
            if (nt < n_tasks) load_all(tn, nxt);
            float acc = 0.f;
            const int lo = u_lo(tc), hi = u_hi(tc);
#pragma unroll
            for (int i = 0; i < ITERS; i++) {
                const int k = lo + sir + i * SPR;
                const float c = tf_b32_step<FMT>(cur[i], k < hi ? k : lo, p, tc.b0, tc.b1, lds, G);
                if (k < hi) acc += c;
            }
            finish(tc, acc);
#pragma unroll
            for (int i = 0; i < ITERS; i++) cur[i] = nxt[i];
            tc = tn;
        }
    } else {
        tf_b32_stage<FMT, SK>(jb, lds);
        for (; task < n_tasks; task += nwaves) {
            const TfB32Task t = tf_b32_task(jb, task * UNITS + unit);
            float acc = 0.f;
            const int lo = u_lo(t), hi = u_hi(t);
            for (int k = lo + sir; t.valid && k < hi; k += SPR) {
                TfB32Regs r;
                tf_b32_load<FMT>(t.col, k, p, r);
                acc += tf_b32_step<FMT>(r, k, p, t.b0, t.b1, lds, G);
            }
            finish(t, acc);
        }
    }
}

// ---------------------------------------------------------------- dispatch

template <int V>
using tf_icb = std::integral_constant<int, V>;

template <int FMT, int SK>
static int tf_b32_launch(TfB32Job jb, tf_stream_t stream) {
    const int G = jb.nb;
    const int lds = tf_b32_lds_bytes(FMT, G);
    if (lds > 65536) return (int)hipErrorInvalidValue;
    // longest unit range of a row (pairs for PAIR, blocks otherwise)
    // (a range of L blocks that starts mid-pair spans (L + 2) / 2 pairs)
    const int L = jb.n_split > 0 ? (G + jb.n_split - 1) / jb.n_split : G;
    const int len = FMT != TF_B32_Q8_PAIR ? L : (jb.n_split > 0 ? (L + 2) / 2 : G / 2);
    int rc = 0;
    auto go = [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        auto fn = tf_b32_kernel<FMT, SK, SPR, IT>;
        const long long tasks = (jb.n_tot + 16 / SPR - 1) / (16 / SPR);
        const int BT = tf_block_threads(512, tasks);
        const int blocks = tf_persistent_blocks((const void*)fn, BT, lds, (int)tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), lds, tf_stream(stream), jb);
        rc = TF_LAUNCH_RESULT();
    };
    if constexpr (FMT == TF_B32_Q8_PAIR) {
        // Quads per row.  Fewer quads, each with more pairs, put more rows
        // on a wave and so more bytes in flight per wave: a wide matrix
        // (the 896 x 151936 lm_head) streams at 0.54 of HBM peak with 4
        // quads per row against 0.40 with 16; a small one is latency-bound
        // and does marginally better with 8.
        const int spr_max = jb.n_tot >= 16384 ? 4 : 8;
        int spr = 4;
        while (spr < len && spr < spr_max) spr *= 2;
        const int its = (len + spr - 1) / spr;
        if (spr == 4 && its <= 4) {
            switch (its) {
            case 1: go(tf_icb<4>{}, tf_icb<1>{}); break;
            case 2: go(tf_icb<4>{}, tf_icb<2>{}); break;
            case 3: go(tf_icb<4>{}, tf_icb<3>{}); break;
            default: go(tf_icb<4>{}, tf_icb<4>{}); break;
            }
        } else if (spr == 8 && its <= 4) {
            switch (its) {
            case 1: go(tf_icb<8>{}, tf_icb<1>{}); break;
            case 2: go(tf_icb<8>{}, tf_icb<2>{}); break;
            case 3: go(tf_icb<8>{}, tf_icb<3>{}); break;
            default: go(tf_icb<8>{}, tf_icb<4>{}); break;
            }
        } else {
            const int i16 = (len + 15) / 16;
            if (i16 == 1) go(tf_icb<16>{}, tf_icb<1>{});
            else if (i16 == 2) go(tf_icb<16>{}, tf_icb<2>{});
            else if (i16 == 3) go(tf_icb<16>{}, tf_icb<3>{});
            else if (i16 == 4) go(tf_icb<16>{}, tf_icb<4>{});
            else go(tf_icb<16>{}, tf_icb<0>{});
        }
    } else {
        if (len <= 4) go(tf_icb<4>{}, tf_icb<0>{});
        else if (len <= 8) go(tf_icb<8>{}, tf_icb<0>{});
        else go(tf_icb<16>{}, tf_icb<0>{});
    }
    return rc;
}

// The pair layout needs an even block count and dword-aligned columns.
static bool tf_q8_0_pair_ok(const uint8_t* const* w, int nw, int nb, int col_bytes) {
    if ((nb & 1) || (col_bytes & 3)) return false;
    for (int i = 0; i < nw; i++)
        if ((uintptr_t)w[i] & 3) return false;
    return true;
}

static int tf_b32_run(int fmt, int sk, TfB32Job& jb, tf_stream_t stream) {
    if (fmt == TF_B32_Q8_PAIR)
        return sk == TF_B32_SRC_Q8 ? tf_b32_launch<TF_B32_Q8_PAIR, TF_B32_SRC_Q8>(jb, stream)
                                   : tf_b32_launch<TF_B32_Q8_PAIR, TF_B32_SRC_F32>(jb, stream);
    if (fmt == TF_B32_Q8_GEN)
        return sk == TF_B32_SRC_Q8 ? tf_b32_launch<TF_B32_Q8_GEN, TF_B32_SRC_Q8>(jb, stream)
                                   : tf_b32_launch<TF_B32_Q8_GEN, TF_B32_SRC_F32>(jb, stream);
    if (fmt == TF_B32_Q8_F32) return tf_b32_launch<TF_B32_Q8_F32, TF_B32_SRC_F32>(jb, stream);
    return tf_b32_launch<TF_B32_Q5_F32, TF_B32_SRC_F32>(jb, stream);
}

// Common argument checks.  block_bytes 34 (Q8_0) or 22 (Q5_0); the weights
// and their columns must be 2-byte aligned (every field is a 16-bit unit).
static bool tf_b32_common_ok(const TfB32Job& jb, int nw, int n_rows, int block_bytes) {
    if (n_rows <= 0 || (n_rows % 32) != 0 || jb.nb != n_rows / 32) return false;
    if (jb.col_bytes < jb.nb * block_bytes || (jb.col_bytes & 1)) return false;
    for (int i = 0; i < nw; i++)
        if (!jb.w[i] || ((uintptr_t)jb.w[i] & 1) || !jb.out[i] || jb.n[i] <= 0) return false;
    return true;
}

static TfB32Job tf_b32_job(const uint8_t* w, float* out, int n_rows, int n_cols, int col_bytes) {
    TfB32Job jb{};
    jb.w[0] = w;
    jb.out[0] = out;
    jb.n[0] = n_cols;
    jb.n_tot = n_cols;
    jb.nb = n_rows / 32;
    jb.col_bytes = col_bytes;
    return jb;
}

static bool tf_b32_q8_src_ok(const int8_t* xq, const float* xd) {
    return xq && xd && ((uintptr_t)xq & 3) == 0;
}

static bool tf_b32_f32_src_ok(const float* x, int fmt) {
    // Q8 quantize-in-LDS reads float2 pairs; the f32 formats read float4
    return x && ((uintptr_t)x & (fmt >= TF_B32_Q8_F32 ? 15 : 7)) == 0;
}

static int tf_b32_rows(int fmt_f32, const uint8_t* w, int sk, const int8_t* xq, const float* xd,
                       const float* x, float* out, int n_rows, int n_cols, int col_bytes,
                       int use_bias, const float* bias, int use_res, const float* residual,
                       int block_bytes, tf_stream_t stream) {
    TfB32Job jb = tf_b32_job(w, out, n_rows, n_cols, col_bytes);
    TF_CHECK_ARG(tf_b32_common_ok(jb, 1, n_rows, block_bytes));
    TF_CHECK_ARG((!use_bias || bias) && use_res >= 0 && use_res <= 2 && (use_res != 1 || residual));
    jb.bias[0] = use_bias ? bias : nullptr;
    jb.use_res = use_res;
    jb.residual = residual;
    int fmt = fmt_f32;
    if (block_bytes == 34 && fmt != TF_B32_Q8_F32)
        fmt = tf_q8_0_pair_ok(jb.w, 1, jb.nb, col_bytes) ? TF_B32_Q8_PAIR : TF_B32_Q8_GEN;
    if (sk == TF_B32_SRC_Q8) {
        TF_CHECK_ARG(tf_b32_q8_src_ok(xq, xd));
        jb.xq = xq;
        jb.xd = xd;
    } else {
        TF_CHECK_ARG(tf_b32_f32_src_ok(x, fmt));
        jb.x = x;
    }
    return tf_b32_run(fmt, sk, jb, stream);
}

static int tf_b32_splitk(int fmt, const uint8_t* w, int sk, const int8_t* xq, const float* xd,
                         const float* x, float* partial, int n_rows, int n_cols, int col_bytes,
                         int n_split, int block_bytes, tf_stream_t stream) {
    TfB32Job jb = tf_b32_job(w, partial, n_rows, n_cols, col_bytes);
    TF_CHECK_ARG(tf_b32_common_ok(jb, 1, n_rows, block_bytes));
    TF_CHECK_ARG(n_split >= 1 && n_split <= 64 && (long long)n_split * n_cols < (1LL << 31));
    jb.n_split = n_split;
    jb.n_tot = n_split * n_cols;
    if (block_bytes == 34 && fmt != TF_B32_Q8_F32)
        fmt = tf_q8_0_pair_ok(jb.w, 1, jb.nb, col_bytes) ? TF_B32_Q8_PAIR : TF_B32_Q8_GEN;
    if (sk == TF_B32_SRC_Q8) {
        TF_CHECK_ARG(tf_b32_q8_src_ok(xq, xd));
        jb.xq = xq;
        jb.xd = xd;
    } else {
        TF_CHECK_ARG(tf_b32_f32_src_ok(x, fmt));
        jb.x = x;
    }
    return tf_b32_run(fmt, sk, jb, stream);
}

static int tf_b32_multi(int fmt, int nw, const uint8_t* const* w, float* const* out,
                        const int* n, const float* x, int n_rows, int col_bytes, int use_bias,
                        const float* const* bias, int block_bytes, tf_stream_t stream) {
    TfB32Job jb{};
    jb.nb = n_rows / 32;
    jb.col_bytes = col_bytes;
    long long tot = 0;
    for (int i = 0; i < nw; i++) {
        jb.w[i] = w[i];
        jb.out[i] = out[i];
        jb.n[i] = n[i];
        jb.bias[i] = use_bias ? bias[i] : nullptr;
        TF_CHECK_ARG(!use_bias || bias[i]);
        tot += n[i] > 0 ? n[i] : 0;
    }
    TF_CHECK_ARG(tf_b32_common_ok(jb, nw, n_rows, block_bytes) && tot < (1LL << 31));
    jb.n_tot = (int)tot;
    if (block_bytes == 34)
        fmt = tf_q8_0_pair_ok(jb.w, nw, jb.nb, col_bytes) ? TF_B32_Q8_PAIR : TF_B32_Q8_GEN;
    TF_CHECK_ARG(tf_b32_f32_src_ok(x, fmt));
    jb.x = x;
    return tf_b32_run(fmt, TF_B32_SRC_F32, jb, stream);
}

// ---------------------------------------------------------------- C ABI

extern "C" int tf_gemv_q8_0_q8(const uint8_t* w, const int8_t* xq, const float* xd, float* out,
                               int n_rows, int n_cols, int col_bytes, int use_bias,
                               const float* bias, int use_res, const float* residual,
                               tf_stream_t stream) {
    return tf_b32_rows(TF_B32_Q8_GEN, w, TF_B32_SRC_Q8, xq, xd, nullptr, out, n_rows, n_cols,
                       col_bytes, use_bias, bias, use_res, residual, 34, stream);
}

extern "C" int tf_gemv_q8_0_f32(const uint8_t* w, const float* x, float* out, int n_rows,
                                int n_cols, int col_bytes, int use_bias, const float* bias,
                                int use_res, const float* residual, tf_stream_t stream) {
    return tf_b32_rows(TF_B32_Q8_GEN, w, TF_B32_SRC_F32, nullptr, nullptr, x, out, n_rows,
                       n_cols, col_bytes, use_bias, bias, use_res, residual, 34, stream);
}

extern "C" int tf_gemv_q5_0_f32(const uint8_t* w, const float* x, float* out, int n_rows,
                                int n_cols, int col_bytes, int use_bias, const float* bias,
                                int use_res, const float* residual, tf_stream_t stream) {
    return tf_b32_rows(TF_B32_Q5_F32, w, TF_B32_SRC_F32, nullptr, nullptr, x, out, n_rows,
                       n_cols, col_bytes, use_bias, bias, use_res, residual, 22, stream);
}

extern "C" int tf_gemv_q8_0_q8_splitk(const uint8_t* w, const int8_t* xq, const float* xd,
                                      float* partial, int n_rows, int n_cols, int col_bytes,
                                      int n_split, tf_stream_t stream) {
    return tf_b32_splitk(TF_B32_Q8_GEN, w, TF_B32_SRC_Q8, xq, xd, nullptr, partial, n_rows,
                         n_cols, col_bytes, n_split, 34, stream);
}

extern "C" int tf_gemv_q8_0_f32_splitk(const uint8_t* w, const float* x, float* partial,
                                       int n_rows, int n_cols, int col_bytes, int n_split,
                                       tf_stream_t stream) {
    return tf_b32_splitk(TF_B32_Q8_F32, w, TF_B32_SRC_F32, nullptr, nullptr, x, partial, n_rows,
                         n_cols, col_bytes, n_split, 34, stream);
}

extern "C" int tf_gemv_q5_0_f32_splitk(const uint8_t* w, const float* x, float* partial,
                                       int n_rows, int n_cols, int col_bytes, int n_split,
                                       tf_stream_t stream) {
    return tf_b32_splitk(TF_B32_Q5_F32, w, TF_B32_SRC_F32, nullptr, nullptr, x, partial, n_rows,
                         n_cols, col_bytes, n_split, 22, stream);
}

extern "C" int tf_gemv_q5_0_qk(const uint8_t* wq, const uint8_t* wk, const float* x, float* q,
                               float* k, int n_rows, int n_q, int n_k, int col_bytes,
                               int use_bias, const float* bq, const float* bk,
                               tf_stream_t stream) {
    const uint8_t* w[2] = {wq, wk};
    float* out[2] = {q, k};
    const int n[2] = {n_q, n_k};
    const float* b[2] = {bq, bk};
    return tf_b32_multi(TF_B32_Q5_F32, 2, w, out, n, x, n_rows, col_bytes, use_bias, b, 22,
                        stream);
}

extern "C" int tf_gemv_q5_0_qkv(const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                                const float* x, float* q, float* k, float* v, int n_rows,
                                int n_q, int n_k, int n_v, int col_bytes, int use_bias,
                                const float* bq, const float* bk, const float* bv,
                                tf_stream_t stream) {
    const uint8_t* w[3] = {wq, wk, wv};
    float* out[3] = {q, k, v};
    const int n[3] = {n_q, n_k, n_v};
    const float* b[3] = {bq, bk, bv};
    return tf_b32_multi(TF_B32_Q5_F32, 3, w, out, n, x, n_rows, col_bytes, use_bias, b, 22,
                        stream);
}

extern "C" int tf_gemv_q8_0_qkv(const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                                const float* x, float* q, float* k, float* v, int n_rows,
                                int n_q, int n_k, int n_v, int col_bytes, int use_bias,
                                const float* bq, const float* bk, const float* bv,
                                tf_stream_t stream) {
    const uint8_t* w[3] = {wq, wk, wv};
    float* out[3] = {q, k, v};
    const int n[3] = {n_q, n_k, n_v};
    const float* b[3] = {bq, bk, bv};
    return tf_b32_multi(TF_B32_Q8_GEN, 3, w, out, n, x, n_rows, col_bytes, use_bias, b, 34,
                        stream);
}
