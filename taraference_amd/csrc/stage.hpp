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
//   q8[320*nb] int8 | d8[G] f32 | ds[G] f32 = d8*sum32(q8) |
//   s16[2G] i32 = per-16 sums of q8 | (optional) xf[256*nb] f32 normalized
//   activation | xs16[2G] f32 = per-16 sums of xf
// The Q4_K x Q8 path reads q8/d8/ds, the Q6_K x Q8 path q8/d8/s16 and the
// Q6_K x f32 path xf/xs16.
// The q8 bytes are padded: value byte o sits at tf_q8_pad(o), 16 bytes of gap
// after every 64, so the GEMV lanes that each read a 64-byte run (lane stride
// 64 B) fall on distinct LDS banks instead of four to a bank.
#pragma once
#include "tf_common.hpp"

__host__ __device__ constexpr int tf_q8_pad(int o) { return o + ((o >> 6) << 4); }
#define TF_Q8_LDS_BYTES(nb) ((nb) * 320)

enum TfSrc { TF_SRC_Q8 = 0, TF_SRC_F32 = 1, TF_SRC_NORM = 2, TF_SRC_FLASH = 3 };

// LDS floats for the merge weights of TF_SRC_FLASH: n_head * (n_split + 1).
#define TF_FLASH_STAGE_W 2048

struct TfAct {
    const int8_t* q8;
    const float* d8;
    const float* ds;
    const int32_t* s16;
    const float* xf;
    const float* xs16;
};

__host__ __device__ constexpr int tf_act_lds_bytes(int nb, bool with_f32) {
    return TF_Q8_LDS_BYTES(nb) + nb * 8 * 4 * 2 + nb * 16 * 4 +
           (with_f32 ? nb * 256 * 4 + nb * 16 * 4 : 0);
}

__device__ __forceinline__ TfAct tf_act_view(uint8_t* lds, int nb) {
    TfAct a;
    a.q8 = reinterpret_cast<const int8_t*>(lds);
    a.d8 = reinterpret_cast<const float*>(lds + TF_Q8_LDS_BYTES(nb));
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
    int n_x;              // TF_SRC_NORM: full row length the RMS is taken over
                          // (>= the 256*nb values staged); 0 = 256*nb.
                          // TF_SRC_FLASH: number of partitions
    int hd;               // TF_SRC_FLASH: head_dim (x = the partial buffer)
    float* dump_f32;      // optional: workgroup 0 also writes the staged row,
    int8_t* dump_q8;      // its Q8 bytes and scales here (float sources)
    float* dump_d8;
};

// Threads per workgroup of the GEMV kernels that stage an activation.  The
// persistent grid runs about one workgroup per CU, so a CU-wide workgroup
// builds the activation image once for all of its waves (resident 256-thread
// workgroups would each rebuild it).  The register budget bounds the size:
// 1024 threads leave 128 VGPRs, 512 leave 256.
__host__ __device__ constexpr int tf_bt_rows(int spr, int sk = TF_SRC_Q8) {
    return sk == TF_SRC_FLASH ? 256 : (spr <= 8 ? 1024 : 512);
}
__host__ __device__ constexpr int tf_bt_pair(int spr) { return spr <= 8 ? 1024 : 256; }
#define TF_BT_QKV 512

// Host side: the kernel instantiation for a source kind.
template <class K>
inline K tf_sk_pick(int kind, K q8, K f32, K norm) {
    return kind == TF_SRC_Q8 ? q8 : (kind == TF_SRC_F32 ? f32 : norm);
}
template <class K>
inline K tf_sk_pick(int kind, K q8, K f32, K norm, K flash) {
    return kind == TF_SRC_FLASH ? flash : tf_sk_pick(kind, q8, f32, norm);
}

// Host-side precondition of a staging source: the f32 sources are read as
// float2 pairs.
inline bool tf_src_ok(const TfActSrc& src) {
    if (src.kind == TF_SRC_Q8) return src.xq && src.xd;
    if ((src.dump_f32 != nullptr) != (src.dump_q8 != nullptr) ||
        (src.dump_q8 != nullptr) != (src.dump_d8 != nullptr) || ((uintptr_t)src.dump_f32 & 7))
        return false;
    if (src.kind == TF_SRC_FLASH)
        return src.x && ((uintptr_t)src.x & 7) == 0 && src.n_x >= 1 && src.n_x <= 64 &&
               (src.hd == 64 || src.hd == 128 || src.hd == 256);
    if (!src.x || ((uintptr_t)src.x & 7) != 0) return false;
    return src.kind != TF_SRC_NORM || (src.norm_w && ((uintptr_t)src.norm_w & 7) == 0);
}


// Build the LDS image.  Must be called by all 256 threads; ends with a
// barrier.  WITH_F32 also keeps the (normalized) f32 activation.
// SK is the source kind (TfSrc), fixed at compile time so that each
// kernel instantiation only holds the staging registers of its own source.
template <bool WITH_F32, int SK>
__device__ __forceinline__ void tf_stage_act(const TfActSrc& src, int nb, uint8_t* lds) {
    int8_t* q8s = reinterpret_cast<int8_t*>(lds);
    float* d8s = reinterpret_cast<float*>(lds + TF_Q8_LDS_BYTES(nb));
    float* dss = d8s + nb * 8;
    int32_t* s16 = reinterpret_cast<int32_t*>(dss + nb * 8);
    float* xf = reinterpret_cast<float*>(s16 + nb * 16);
    float* xs16 = xf + nb * 256;
    const int groups = nb * 8;
    if constexpr (SK == TF_SRC_Q8) {
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
            reinterpret_cast<tf_u32x4*>(q8s + tf_q8_pad(g * 32))[0] = a;
            reinterpret_cast<tf_u32x4*>(q8s + tf_q8_pad(g * 32))[1] = b;
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
    } else {
        // F32 / NORM / FLASH.  The quantization runs on value pairs: with NW
        // waves and SPAN = 128 NW, at step k lane L of wave w holds values
        // e0 = SPAN k + 128 w + 2 L and e0 + 1, so the 16 lanes of a DPP row
        // hold one whole 32-value group and every group reduction is a DPP
        // row operation (tf_q8_pair).
        const int n = nb * 256;
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int NW = blockDim.x >> 6, SPAN = 128 * NW;
        const int m = lane & 15;
        // Quantize four value pairs (four steps) and write the LDS image.
        // Nothing branches: a step with e0 < 0 (past the row) and lanes that
        // own no scale / sum store to a dummy LDS slot instead, so the four
        // independent chains (DPP reductions, divisions) interleave.
        __shared__ __align__(16) int tf_dummy[4];
        auto emit4 = [&](const int (&e0)[4], const float (&x0)[4], const float (&x1)[4]) {
            TfQ8Pair r[4];
#pragma unroll
            for (int k = 0; k < 4; k++) r[k] = tf_q8_pair<WITH_F32>(x0[k], x1[k]);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const bool ok = e0[k] >= 0;
                const int e = ok ? e0[k] : 0;
                const int g = e >> 5, half = m >> 3;
                uint16_t* pq = ok ? reinterpret_cast<uint16_t*>(q8s + tf_q8_pad(e))
                                  : reinterpret_cast<uint16_t*>(tf_dummy);
                *pq = (uint16_t)((r[k].q0 & 0xff) | ((r[k].q1 & 0xff) << 8));
                int* ps = (ok && (m & 7) == 0) ? s16 + 2 * g + half : tf_dummy + 1;
                *ps = r[k].s_half;
                const bool own = ok && m == 0;
                float* pd = own ? d8s + g : reinterpret_cast<float*>(tf_dummy + 2);
                float* pds = own ? dss + g : reinterpret_cast<float*>(tf_dummy + 3);
                *pd = r[k].d;
                *pds = r[k].d * (float)(r[k].s_half + r[k].s_other);
                if (WITH_F32) {
                    float2* px = ok ? reinterpret_cast<float2*>(xf + e)
                                    : reinterpret_cast<float2*>(tf_dummy);
                    *px = make_float2(x0[k], x1[k]);
                    float* pfs = (ok && (m & 7) == 0) ? xs16 + 2 * g + half
                                                      : reinterpret_cast<float*>(tf_dummy + 1);
                    *pfs = r[k].f_half;
                }
                if constexpr (SK == TF_SRC_FLASH) {
                    if (src.dump_f32 && blockIdx.x == 0 && ok) {  // merged row (tests)
                        *reinterpret_cast<float2*>(src.dump_f32 + e) = make_float2(x0[k], x1[k]);
                        src.dump_q8[e] = (int8_t)r[k].q0;
                        src.dump_q8[e + 1] = (int8_t)r[k].q1;
                        if (m == 0) src.dump_d8[g] = r[k].d;
                    }
                }
            }
        };
        // Every workgroup reads the same row at the same time; starting each
        // one at a different step spreads the requests over the L2 channels.
        // Step v of this workgroup is row step (v + rot) % S.
        const int S = (n + SPAN - 1) / SPAN;
        const int rot = blockIdx.x % S;
        if constexpr (SK == TF_SRC_FLASH) {
            // Log-sum-exp merge of split-KV partials (m, l, O[hd]) for the
            // n/hd heads of the row, in the reference's order
            // (attn/flash.cu:222-255): M = max_s m_s, a_s = e^(m_s - M),
            // l = sum_s a_s l_s and o[d] = sum_s a_s O_s[d] in split order,
            // out = o / max(l, 1e-20).
            const float* part = src.x;
            const int ns = src.n_x, hd = src.hd, po = hd + 2, nh = n / hd;
            __shared__ float fw[TF_FLASH_STAGE_W];
            float* Ls = fw + nh * ns;
            // wave w merges heads w, w + NW, ...; all their (m, l) loads
            // are issued first (nh <= 8 NW)
            float mv[8], lv[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {  // loads from clamped addresses: no branches
                const int h = wave + NW * j;
                const bool live = h < nh && lane < ns;
                const float* ph = part + (live ? ((size_t)h * ns + lane) * po : 0);
                const float m0 = ph[0], l0 = ph[1];
                mv[j] = live ? m0 : -1e30f;
                lv[j] = live ? l0 : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int h = wave + NW * j;
                if (h >= nh) break;  // wave-uniform
                const float M = tf_wave_max(mv[j]);
                const float av = lane < ns ? __expf(mv[j] - M) : 0.f;
                if (lane < ns) fw[h * ns + lane] = av;
                float L = 0.f;
                for (int s2 = 0; s2 < ns; s2++)
                    L = fmaf(tf_readlane(av, s2), tf_readlane(lv[j], s2), L);
                if (lane == 0) Ls[h] = L;
            }
            __syncthreads();
            // steps in groups of 4, splits in chunks of 8: 32 value pairs in
            // flight per thread, loaded from clamped addresses (no branches)
            for (int v0 = 0; v0 < S; v0 += 4) {
                int e0k[4];
                bool okk[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    int st = v0 + k + rot;
                    if (st >= S) st -= S;
                    okk[k] = v0 + k < S && SPAN * st + 128 * wave < n;
                    e0k[k] = okk[k] ? SPAN * st + 128 * wave + 2 * lane : 0;
                }
                float2 acc[4];
#pragma unroll
                for (int k = 0; k < 4; k++) acc[k] = make_float2(0.f, 0.f);
                for (int s0 = 0; s0 < ns; s0 += 8) {
                    float2 o[8][4];
#pragma unroll
                    for (int u = 0; u < 8; u++)
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            const int h = e0k[k] / hd, d = e0k[k] - h * hd;
                            const bool ok = s0 + u < ns && okk[k];
                            o[u][k] = *reinterpret_cast<const float2*>(
                                part + (ok ? ((size_t)h * ns + s0 + u) * po + 2 + d : 2));
                        }
#pragma unroll
                    for (int u = 0; u < 8; u++)
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            if (s0 + u < ns && okk[k]) {  // uniform per wave
                                const float a = fw[(e0k[k] / hd) * ns + s0 + u];
                                acc[k].x = fmaf(a, o[u][k].x, acc[k].x);
                                acc[k].y = fmaf(a, o[u][k].y, acc[k].y);
                            }
                        }
                }
                int ek[4];
                float q0[4], q1[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float den = fmaxf(Ls[e0k[k] / hd], 1e-20f);
                    ek[k] = okk[k] ? e0k[k] : -1;
                    q0[k] = acc[k].x / den;
                    q1[k] = acc[k].y / den;
                }
                emit4(ek, q0, q1);
            }
        } else {
            // F32 / NORM.  NORM first forms the sum of squares in the
            // reference's order (per-thread strided fused multiply-adds over
            // x[t + 256j], then the halving tree) over the full row length,
            // exactly as tf_norm_quant does, so the Q8 bytes are identical.
            constexpr bool norm = SK == TF_SRC_NORM;
            const int n_x = (norm && src.n_x > 0) ? src.n_x : n;
            __shared__ float red[256];
            // NORM rows (the model width) are short: 4-step chunks of x and
            // w.  F32 rows (the FFN width) are long: 8-step chunks of x, the
            // next chunk's loads in flight while one is quantized.
            // NORM rows (the model width, <= 4096 here) and F32 rows (the FFN
            // width) are read in chunks of STEPS value-pair steps whose loads
            // are all in flight together; the addresses are clamped rather
            // than branched around, so nothing serializes them.
            constexpr int STEPS = norm ? 8 : 16;
            float2 xv[STEPS], wv[norm ? STEPS : 1];
            // offset of virtual step v in the row, or -1 past the row / wave span
            auto vstep_e0 = [&](int v) {
                const int st = v + rot >= S ? v + rot - S : v + rot;
                const bool ok = v < S && SPAN * st + 128 * wave < n;
                return ok ? SPAN * st + 128 * wave + 2 * lane : -1;
            };
            auto load_chunk = [&](int v0) {
#pragma unroll
                for (int k = 0; k < STEPS; k++) {
                    const int e0 = vstep_e0(v0 + k);
                    const int ec = e0 < 0 ? 0 : e0;
                    xv[k] = *reinterpret_cast<const float2*>(src.x + ec);
                    if constexpr (norm) wv[k] = *reinterpret_cast<const float2*>(src.norm_w + ec);
                }
            };
            load_chunk(0);
            float scale = 1.f;
            if constexpr (norm) {
                // the reference's 256 strided partial sums: threads 0-255
                float local = 0.f;
                for (int j0 = 0; tid < 256 && j0 < n_x; j0 += 8 * 256) {
                    float v[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const int i = j0 + 256 * u + tid;
                        const float xi = src.x[i < n_x ? i : 0];
                        v[u] = i < n_x ? xi : 0.f;
                    }
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        if (j0 + 256 * u + tid < n_x) local = fmaf(v[u], v[u], local);
                }
                if (tid < 256) red[tid] = local;
                __syncthreads();
                if (tid < 128) red[tid] += red[tid + 128];
                __syncthreads();
                if (tid < 64) {
                    float v = red[tid] + red[tid + 64];
                    v += __shfl_down(v, 32, 64);
                    v += __shfl_down(v, 16, 64);
                    v += __shfl_down(v, 8, 64);
                    v += __shfl_down(v, 4, 64);
                    v += __shfl_down(v, 2, 64);
                    v += __shfl_down(v, 1, 64);
                    if (tid == 0) red[0] = 1.0f / sqrtf(v / (float)n_x + src.eps);
                }
                __syncthreads();
                scale = red[0];
            }
            for (int v0 = 0; v0 < S; v0 += STEPS) {
                if (v0) load_chunk(v0);
#pragma unroll
                for (int k4 = 0; k4 < STEPS; k4 += 4) {
                    if (v0 + k4 >= S) break;  // block-uniform
                    int ek[4];
                    float q0[4], q1[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        ek[k] = vstep_e0(v0 + k4 + k);
                        q0[k] = xv[k4 + k].x;
                        q1[k] = xv[k4 + k].y;
                        if constexpr (norm) {
                            q0[k] = q0[k] * scale * wv[k4 + k].x;
                            q1[k] = q1[k] * scale * wv[k4 + k].y;
                        }
                    }
                    emit4(ek, q0, q1);
                }
            }
        }
    }
    __syncthreads();
}
