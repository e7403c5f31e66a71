// Prefill (n_tok > 1) for gfx950: Q4_K / Q6_K GEMMs on the matrix cores and
// causal tiled attention.
//
// Replaces kernels/gemm.cu gemm_q4_k (:6) and gemm_q6_k (:69) (matmul.rs:1269
// gemm) and kernels/attn/fast_v2.cu attn_fast_v2 / attn_fast_v2_d (:12, :103).
//
// GEMM: out[t][j] = sum_k W[k][j] x[t][k] with x f32.  The reference
// dequantizes each weight to f32 and accumulates in fp32; the result must
// stay within fp32 GEMV accuracy, so the matrix cores are used as follows.
// A K-quant weight is (scale of its sub-block) x (small integer):
//   Q4_K  W = d*sc_s*q - dmin*m_s, q in 0..15, sub-blocks of 32,
//   Q6_K  W = d*sc_s*(q - 32),     q - 32 in -32..31, sub-blocks of 16.
// Small integers are exact in bf16, and x is split exactly into three bf16
// parts, x = x0 + x1 + x2 (each the truncation of the remainder, so the
// error is below 2^-21 |x|).  Per sub-block the matrix cores form sum(q x)
// with fp32 accumulation, one MFMA per part (Q4_K: v_mfma_f32_16x16x32_bf16,
// one 32-deep step per sub-block; Q6_K: v_mfma_f32_16x16x16_bf16, one
// 16-deep step per sub-block), and the fp32 epilogue applies the scales:
//   acc += (d*sc_s) * sum(q x) - (dmin*m_s) * sum(x)      (Q4_K)
//   acc += (d*sc_s) * sum((q-32) x)                        (Q6_K).
// The products of the matrix cores are exact; only the fp32 summation order
// differs from the reference's.
//
// Tiling: a workgroup (4 waves) owns 128 output columns x 32 tokens; a wave
// owns 32 columns (two 16-column tiles) x 32 tokens (two 16-token tiles).
// Per 256-value super-block the workgroup stages x in LDS already split into
// its three bf16 planes (once per workgroup, with the per-group sums of x)
// and the per-sub-block scales of its columns; each wave reads its own
// columns' quant bytes straight from global memory.  All global loads of
// super-block sb + 1 are issued before the MFMAs of super-block sb.  Consecutive workgroups share columns (token tiles are
// the fast grid dimension), so a column's bytes are re-read from L2.
//
// MFMA operand layouts (lane l, g = l / 16), A rows = output columns,
// B columns = tokens, C[i][j] with j = l % 16, i = 4g .. 4g+3:
//   16x16x16: A[l % 16][4g .. 4g+3], B[4g .. 4g+3][l % 16];
//   16x16x32: A[l % 16][8g .. 8g+7], B[8g .. 8g+7][l % 16].
#include "dequant.hpp"
#include "prefill.hpp"
#include "tf_common.hpp"
#include "tf_host.hpp"

typedef short tf_bf16x4 __attribute__((ext_vector_type(4)));
typedef float tf_f32x4 __attribute__((ext_vector_type(4)));

#define TF_PF_COLS 128  // output columns per workgroup
// s_waitcnt immediate (gfx9 encoding): vmcnt 0, expcnt and lgkmcnt unchanged
#define TF_VMCNT0 0x0F70
#define TF_PF_TOKS 32   // tokens per workgroup

// Three-part bf16 split of four floats (truncation; every remainder exact).
struct TfSplit3 {
    tf_bf16x4 p[3];
};
__device__ __forceinline__ TfSplit3 tf_split3(float4 v) {
    TfSplit3 s;
    float r[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int part = 0; part < 3; part++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t b = __float_as_uint(r[i]) & 0xffff0000u;
            s.p[part][i] = (short)(b >> 16);
            r[i] -= __uint_as_float(b);
        }
    }
    return s;
}

// bf16 bits of a small integer (exact).
__device__ __forceinline__ short tf_bf16_int(int q) {
    return (short)(__float_as_uint((float)q) >> 16);
}

__device__ __forceinline__ uint32_t tf_pf_u16x2(const uint8_t* p) {
    const TF_GAS uint16_t* s = (const TF_GAS uint16_t*)p;
    return s[0] | ((uint32_t)s[1] << 16);
}

// Q4_K 6-bit scale and min of sub-block j (the GGML packing).
__device__ __forceinline__ void tf_pf_scale_min(const uint8_t* s12, int j, int& sc, int& m) {
    if (j < 4) {
        sc = s12[j] & 63;
        m = s12[j + 4] & 63;
    } else {
        sc = (s12[j + 4] & 0xF) | ((s12[j - 4] >> 6) << 4);
        m = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
    }
}

typedef __bf16 tf_bf16x8 __attribute__((ext_vector_type(8)));
typedef short tf_s16x8 __attribute__((ext_vector_type(8)));

// Per-lane quant bytes of one column for one super-block.
//   Q4_K (16x16x32 steps, K step = sub-block s, lane values 32 s + 8g .. +7):
//     w[2c], w[2c+1] = qs bytes 32c + 8g .. +7 (sub-blocks 2c low nibbles,
//     2c+1 high nibbles).
//   Q6_K (16x16x16 steps, K step = sub-block st, lane values 16 st + 4g .. +3):
//     w[0..7] = ql dwords (n, qd&1, half), w[8..11] = qh dwords (n, half).
template <bool Q6>
struct TfPfCol {
    uint32_t w[Q6 ? 12 : 8];
};

template <bool Q6>
__device__ __forceinline__ void tf_pf_load_col(const uint8_t* blk, int g, TfPfCol<Q6>& c) {
    if constexpr (!Q6) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const tf_u32x2 v = *(const TF_GAS tf_u32x2*)(blk + 16 + 32 * i + 8 * g);
            c.w[2 * i] = v.x;
            c.w[2 * i + 1] = v.y;
        }
    } else {
        // raw 210-byte blocks are 2-byte aligned: 16-bit loads
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int n = i >> 2, odd = (i >> 1) & 1, half = i & 1;
            c.w[i] = tf_pf_u16x2(blk + 64 * n + 32 * odd + 16 * half + 4 * g);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = i >> 1, half = i & 1;
            c.w[8 + i] = tf_pf_u16x2(blk + 128 + 32 * n + 16 * half + 4 * g);
        }
    }
}

// Q4_K A operand of sub-block s: 8 codes as bf16.
__device__ __forceinline__ tf_s16x8 tf_pf_a4(const TfPfCol<false>& c, int s) {
    tf_s16x8 a;
    const int sh = 4 * (s & 1);
    const uint32_t lo = c.w[2 * (s >> 1)] >> sh, hi = c.w[2 * (s >> 1) + 1] >> sh;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[i] = tf_bf16_int((lo >> (8 * i)) & 15);
        a[4 + i] = tf_bf16_int((hi >> (8 * i)) & 15);
    }
    return a;
}

// Q6_K A operand of sub-block st: 4 signed codes as bf16.
__device__ __forceinline__ tf_bf16x4 tf_pf_a6(const TfPfCol<true>& c, int st) {
    tf_bf16x4 a;
    const int n = st >> 3, qd = (st & 7) >> 1, half = st & 1;
    const uint32_t ql = c.w[n * 4 + (qd & 1) * 2 + half] >> (4 * (qd >> 1));
    const uint32_t qh = c.w[8 + n * 2 + half] >> (2 * qd);
#pragma unroll
    for (int i = 0; i < 4; i++)
        a[i] = tf_bf16_int((int)(((ql >> (8 * i)) & 15) | (((qh >> (8 * i)) & 3) << 4)) - 32);
    return a;
}

__device__ __forceinline__ tf_f32x4 tf_mfma32(tf_s16x8 a, tf_s16x8 b, tf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(tf_bf16x8, a),
                                                   __builtin_bit_cast(tf_bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ tf_f32x4 tf_mfma16(tf_bf16x4 a, tf_bf16x4 b, tf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

#ifdef TF_GEMM_STAMPS
__device__ unsigned long long tf_gemm_stamps[256];
#define TF_GSTAMP(k)                                                                    \
    do {                                                                               \
        if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0 && (k) < 256)       \
            tf_gemm_stamps[(k)] = __builtin_amdgcn_s_memrealtime();                    \
    } while (0)
extern "C" int tf_gemm_debug_stamps(unsigned long long* host) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(tf_gemm_stamps), sizeof(tf_gemm_stamps));
}
#else
#define TF_GSTAMP(k) \
    do {             \
    } while (0)
#endif

// LDS image of x for one super-block: 3 bf16 planes x 32 tokens x 256
// values, rows of TF_PF_ROW bytes (16 bytes of padding: the 16 rows a
// fragment read touches start on distinct banks).
#define TF_PF_ROW 528
#define TF_PF_XBYTES (3 * TF_PF_TOKS * TF_PF_ROW)

template <bool Q6>
__global__ __launch_bounds__(256) void tf_gemm_kq_kernel(const uint8_t* __restrict__ w,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ out, int n_rows,
                                                          int n_cols, int col_bytes, int n_tok,
                                                          int accumulate, int n_split,
                                                          long long split_stride) {
    constexpr int NSUB = Q6 ? 16 : 8;
    constexpr int BLK = Q6 ? 210 : 144;
    __shared__ __align__(16) uint8_t xp[TF_PF_XBYTES];
    __shared__ float xsum[Q6 ? 1 : TF_PF_TOKS * 8];
    __shared__ __align__(16) float scl[NSUB * TF_PF_COLS];
    __shared__ __align__(16) float mnl[Q6 ? 1 : 8 * TF_PF_COLS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    // XCD-aware tile order: workgroups go round-robin to the 8 XCDs, so XCD
    // k = blockIdx.x % 8 takes the contiguous tile range [k per, (k+1) per)
    // (token tiles fastest): a column tile's weights are fetched into one
    // XCD's L2 and reused there by all its token tiles.
    const int ntx = (n_tok + TF_PF_TOKS - 1) / TF_PF_TOKS;
    const int n_tiles = ntx * ((n_cols + TF_PF_COLS - 1) / TF_PF_COLS);
    const int per = (n_tiles + 7) >> 3;
    const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (tile >= n_tiles) return;  // workgroup-uniform, before any barrier
    const int t0 = (tile % ntx) * TF_PF_TOKS;
    const int c0 = (tile / ntx) * TF_PF_COLS;
    const int nb = n_rows / 256;
    // split z of n_split takes super-blocks [sb_lo, sb_hi) into its own slice
    const int z = blockIdx.z;
    const int sb_lo = (int)((long long)z * nb / n_split);
    const int sb_hi = (int)((long long)(z + 1) * nb / n_split);
    out += (size_t)z * (size_t)split_stride;
    // this lane's A columns (one per 16-column tile), clamped for loads
    int colA[2];
    for (int ct = 0; ct < 2; ct++) {
        const int c = c0 + 32 * wave + 16 * ct + l16;
        colA[ct] = c < n_cols ? c : n_cols - 1;
    }
    tf_f32x4 acc[2][2];
    for (int ct = 0; ct < 2; ct++)
        for (int tt = 0; tt < 2; tt++) acc[ct][tt] = tf_f32x4{0.f, 0.f, 0.f, 0.f};

    // Software pipeline over super-blocks: the global loads of super-block
    // sb + 1 (this lane's quant bytes, this thread's x values, the scale
    // header of one column) are issued before the MFMAs of super-block sb,
    // and written to LDS after them.
    const int xt = tid >> 3, xs = tid & 7;  // staging: token xt, 32-value group xs
    const bool xlive = t0 + xt < n_tok;
    const float* xrow = x + (size_t)(xlive ? t0 + xt : 0) * n_rows + 32 * xs;
    const int hc = c0 + tid < n_cols ? c0 + tid : n_cols - 1;  // header column (tid < 128)
    const uint8_t* hcol = w + (size_t)hc * col_bytes;
    auto load_x = [&](int sb, float4 (&xr)[8]) {
#pragma unroll
        for (int k = 0; k < 8; k++) xr[k] = *reinterpret_cast<const float4*>(xrow + sb * 256 + 4 * k);
    };
    // Q4_K header: d | dmin, 12 scale bytes (4-byte aligned 144-byte blocks);
    // Q6_K: 16 int8 scales and d (2-byte aligned raw blocks)
    auto load_hdr = [&](int sb, uint32_t (&hd)[5]) {
        const uint8_t* blk = hcol + (size_t)sb * BLK;
        if (tid >= TF_PF_COLS) return;
        if constexpr (!Q6) {
            const tf_u32x4 v = tf_ld16_a4(blk);
            hd[0] = v.x;
            hd[1] = v.y;
            hd[2] = v.z;
            hd[3] = v.w;
            hd[4] = 0;
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) hd[i] = tf_pf_u16x2(blk + 192 + 4 * i);
            hd[4] = tf_gld(reinterpret_cast<const uint16_t*>(blk + 208));
        }
    };
    auto store_x = [&](const float4 (&xr)[8]) {
        float gs = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = xlive ? xr[k] : make_float4(0.f, 0.f, 0.f, 0.f);
            gs += (v.x + v.y) + (v.z + v.w);
            const TfSplit3 sp = tf_split3(v);
#pragma unroll
            for (int pl = 0; pl < 3; pl++)
                *reinterpret_cast<tf_bf16x4*>(xp + (pl * TF_PF_TOKS + xt) * TF_PF_ROW +
                                              2 * (32 * xs + 4 * k)) = sp.p[pl];
        }
        if constexpr (!Q6) xsum[xt * 8 + xs] = gs;
    };
    auto store_hdr = [&](const uint32_t (&hd)[5]) {
        if (tid >= TF_PF_COLS) return;
        if constexpr (!Q6) {
            const float d = tf_h2f(hd[0]), dmin = tf_h2f(hd[0] >> 16);
            uint8_t s12[12];
#pragma unroll
            for (int i = 0; i < 12; i++) s12[i] = (uint8_t)(hd[1 + i / 4] >> (8 * (i % 4)));
#pragma unroll
            for (int s = 0; s < 8; s++) {
                int sc, m;
                tf_pf_scale_min(s12, s, sc, m);
                scl[s * TF_PF_COLS + tid] = d * (float)sc;
                mnl[s * TF_PF_COLS + tid] = dmin * (float)m;
            }
        } else {
            const float d = tf_h2f(hd[4]);
#pragma unroll
            for (int s = 0; s < 16; s++)
                scl[s * TF_PF_COLS + tid] = d * (float)(int8_t)(hd[s / 4] >> (8 * (s % 4)));
        }
    };

    TfPfCol<Q6> wc[2], wn[2];
    float4 xr[8];
    uint32_t hd[5];
    for (int ct = 0; ct < 2; ct++)
        tf_pf_load_col<Q6>(w + (size_t)colA[ct] * col_bytes + (size_t)sb_lo * BLK, g, wc[ct]);
    load_x(sb_lo, xr);
    load_hdr(sb_lo, hd);
    // Nothing may be pending at loop entry: the wait-count insertion merges
    // the loop header's state over both edges, and a prologue load still in
    // flight into wc would make every iteration wait for its own prefetch
    // of the next super-block before the first use of wc.
    __builtin_amdgcn_s_waitcnt(TF_VMCNT0);
    TF_GSTAMP(0);
    for (int sb = sb_lo; sb < sb_hi; sb++) {
        TF_GSTAMP(1 + 4 * sb);
        __syncthreads();  // the previous super-block's LDS reads are done
        TF_GSTAMP(2 + 4 * sb);
        store_x(xr);
        store_hdr(hd);
        __syncthreads();
        TF_GSTAMP(3 + 4 * sb);
        if (sb + 1 < sb_hi) {  // workgroup-uniform
            for (int ct = 0; ct < 2; ct++)
                tf_pf_load_col<Q6>(w + (size_t)colA[ct] * col_bytes + (size_t)(sb + 1) * BLK, g,
                                   wn[ct]);
            load_x(sb + 1, xr);
            load_hdr(sb + 1, hd);
        }
        for (int s = 0; s < NSUB; s++) {
            tf_f32x4 part[2][2];
            if constexpr (!Q6) {
                tf_s16x8 b[2][3];
                for (int tt = 0; tt < 2; tt++)
                    for (int pl = 0; pl < 3; pl++)
                        b[tt][pl] = *reinterpret_cast<const tf_s16x8*>(
                            xp + (pl * TF_PF_TOKS + 16 * tt + l16) * TF_PF_ROW + 2 * (32 * s + 8 * g));
                for (int ct = 0; ct < 2; ct++) {
                    const tf_s16x8 a = tf_pf_a4(wc[ct], s);
                    for (int tt = 0; tt < 2; tt++) {
                        tf_f32x4 c = tf_mfma32(a, b[tt][0], tf_f32x4{0.f, 0.f, 0.f, 0.f});
                        c = tf_mfma32(a, b[tt][1], c);
                        part[ct][tt] = tf_mfma32(a, b[tt][2], c);
                    }
                }
            } else {
                tf_bf16x4 b[2][3];
                for (int tt = 0; tt < 2; tt++)
                    for (int pl = 0; pl < 3; pl++)
                        b[tt][pl] = *reinterpret_cast<const tf_bf16x4*>(
                            xp + (pl * TF_PF_TOKS + 16 * tt + l16) * TF_PF_ROW + 2 * (16 * s + 4 * g));
                for (int ct = 0; ct < 2; ct++) {
                    const tf_bf16x4 a = tf_pf_a6(wc[ct], s);
                    for (int tt = 0; tt < 2; tt++) {
                        tf_f32x4 c = tf_mfma16(a, b[tt][0], tf_f32x4{0.f, 0.f, 0.f, 0.f});
                        c = tf_mfma16(a, b[tt][1], c);
                        part[ct][tt] = tf_mfma16(a, b[tt][2], c);
                    }
                }
            }
            for (int ct = 0; ct < 2; ct++) {
                // scales of C rows 4g..4g+3 = columns 16 ct + 4g + r of this wave
                const float4 sc4 = *reinterpret_cast<const float4*>(
                    scl + s * TF_PF_COLS + 32 * wave + 16 * ct + 4 * g);
                float4 mn4 = make_float4(0.f, 0.f, 0.f, 0.f);
                if constexpr (!Q6)
                    mn4 = *reinterpret_cast<const float4*>(
                        mnl + s * TF_PF_COLS + 32 * wave + 16 * ct + 4 * g);
                const float scv[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
                const float mnv[4] = {mn4.x, mn4.y, mn4.z, mn4.w};
                for (int tt = 0; tt < 2; tt++) {
                    const float xs_s = Q6 ? 0.f : xsum[(16 * tt + l16) * 8 + (s & 7)];
                    for (int r = 0; r < 4; r++) {
                        float v = acc[ct][tt][r] + scv[r] * part[ct][tt][r];
                        if constexpr (!Q6) v -= mnv[r] * xs_s;
                        acc[ct][tt][r] = v;
                    }
                }
            }
        }
        for (int ct = 0; ct < 2; ct++) wc[ct] = wn[ct];
    }
    TF_GSTAMP(4 * nb + 1);
    // C rows 4g..4g+3 -> columns, C column l16 -> token
    for (int ct = 0; ct < 2; ct++) {
        const int cb = c0 + 32 * wave + 16 * ct + 4 * g;
        for (int tt = 0; tt < 2; tt++) {
            const int t = t0 + 16 * tt + l16;
            if (t >= n_tok) continue;
            float* o = out + (size_t)t * n_cols + cb;
            // accumulate: out += W x (the residual stream), one rounding
            if (cb + 3 < n_cols && ((n_cols & 3) == 0)) {
                float4 v = make_float4(acc[ct][tt][0], acc[ct][tt][1], acc[ct][tt][2],
                                       acc[ct][tt][3]);
                if (accumulate) {
                    const float4 o0 = *reinterpret_cast<const float4*>(o);
                    v = make_float4(o0.x + v.x, o0.y + v.y, o0.z + v.z, o0.w + v.w);
                }
                *reinterpret_cast<float4*>(o) = v;
            } else {
                for (int r = 0; r < 4; r++)
                    if (cb + r < n_cols) o[r] = accumulate ? o[r] + acc[ct][tt][r] : acc[ct][tt][r];
            }
        }
    }
}

// ------------------------------------------------- Q4_K GEMM, f16 operands
//
// The Q4_K GEMM on v_mfma_f32_16x16x32_f16 with the sub-block scale folded
// into the A operand, so a whole super-block accumulates in the matrix
// cores and the scales are applied once per super-block:
//   A = sc_s * q   (integer <= 63 * 15 = 945: exact in f16),
//   x = 2^-e (h0 + h1), h0 = f16(x 2^e), h1 = f16(x 2^e - h0), with e per
//       (token, super-block) chosen so max |x 2^e| lies in [2^14, 2^15);
//       the split keeps 22 bits (|x - 2^-e (h0 + h1)| <= 2^-23 |x|, plus
//       2^-25 absolute in the subnormal range of h1),
//   P = sum_k A h (two MFMAs per K step, exact products, fp32 sums),
//   M = sum_s m_s S_s with S_s = 2^(e-5) sum(x over sub-block s) split into
//       two f16 parts (one v_mfma_f32_16x16x16_f16 pair, K = 8 padded to 16),
//   acc += d 2^-e P - dmin 2^(5-e) M.
// Against the reference's fp32 product the difference is the split error
// (2^-23 relative per term) and the fp32 summation order.
//
// A is built from the packed nibbles without conversions: (b & 0x000F000F)
// | 0x64006400 holds 1024 + q of bytes 0 and 2 as two f16, and one packed
// fma with (sc, -1024 sc) gives sc q (fused: the product is not rounded).
// A lane's 8 K values therefore come in the byte order 0 2 1 3 4 6 5 7, and
// x is staged in LDS in that same order within each group of 8.

typedef _Float16 tf_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 tf_h4v __attribute__((ext_vector_type(4)));
typedef _Float16 tf_h8 __attribute__((ext_vector_type(8)));

#define TF_PH_ROW 528  // 256 f16 + 16 bytes of padding
#define TF_PH_XBYTES (2 * TF_PF_TOKS * TF_PH_ROW)
#ifndef TF_PH_WAVES
#define TF_PH_WAVES __attribute__((amdgpu_waves_per_eu(3)))
#endif

__device__ __forceinline__ uint32_t tf_ph_pk(float a, float b) {
    const tf_h2 h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}

// A operand (8 values sc q) from two qs dwords, nibble shift sh (0 or 4).
// (v & mask) | magic in one instruction; gfx9 VOP3 takes no literal, so the
// mask comes in a VGPR and the magic in an SGPR.
__device__ __forceinline__ uint32_t tf_ph_and_or(uint32_t v, uint32_t mask_v) {
    uint32_t r;
    asm volatile("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(mask_v), "s"(0x64006400u));
    return r;
}
__device__ __forceinline__ tf_h8 tf_ph_a(uint32_t lo, uint32_t hi, int sh, uint2 scn,
                                         uint32_t mask_v) {
    const tf_h2 s2 = __builtin_bit_cast(tf_h2, scn.x), n2 = __builtin_bit_cast(tf_h2, scn.y);
    const uint32_t t[4] = {tf_ph_and_or(lo >> sh, mask_v), tf_ph_and_or(lo >> (sh + 8), mask_v),
                           tf_ph_and_or(hi >> sh, mask_v), tf_ph_and_or(hi >> (sh + 8), mask_v)};
    tf_h8 a;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const tf_h2 v = __builtin_elementwise_fma(__builtin_bit_cast(tf_h2, t[i]), s2, n2);
        a[2 * i] = v[0];
        a[2 * i + 1] = v[1];
    }
    return a;
}

__global__ __launch_bounds__(256) TF_PH_WAVES void tf_gemm_q4k_h_kernel(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ x,
                                                            float* __restrict__ out, int n_rows,
                                                            int n_cols, int col_bytes, int n_tok,
                                                            int accumulate, int n_split,
                                                            long long split_stride) {
    __shared__ __align__(16) uint8_t xp[TF_PH_XBYTES];      // [part][token][256] f16
    __shared__ __align__(16) _Float16 xsm[2 * TF_PF_TOKS * 8];  // [part][token][sub-block]
    __shared__ float xinv[TF_PF_TOKS];                       // 2^-e per token
    __shared__ __align__(16) uint2 scn[8 * TF_PF_COLS];      // [sub-block][column] (sc, -1024 sc)
    __shared__ __align__(16) _Float16 mh[TF_PF_COLS * 8];    // [column][sub-block] m
    __shared__ __align__(16) float dd[TF_PF_COLS], dm[TF_PF_COLS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    // XCD-aware tile order: workgroups go round-robin to the 8 XCDs, so XCD
    // k = blockIdx.x % 8 takes the contiguous tile range [k per, (k+1) per)
    // (token tiles fastest): a column tile's weights are fetched into one
    // XCD's L2 and reused there by all its token tiles.
    const int ntx = (n_tok + TF_PF_TOKS - 1) / TF_PF_TOKS;
    const int n_tiles = ntx * ((n_cols + TF_PF_COLS - 1) / TF_PF_COLS);
    const int per = (n_tiles + 7) >> 3;
    const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (tile >= n_tiles) return;  // workgroup-uniform, before any barrier
    const int t0 = (tile % ntx) * TF_PF_TOKS;
    const int c0 = (tile / ntx) * TF_PF_COLS;
    const int nb = n_rows / 256;
    const int z = blockIdx.z;
    const int sb_lo = (int)((long long)z * nb / n_split);
    const int sb_hi = (int)((long long)(z + 1) * nb / n_split);
    out += (size_t)z * (size_t)split_stride;
    int colA[2];
    for (int ct = 0; ct < 2; ct++) {
        const int c = c0 + 32 * wave + 16 * ct + l16;
        colA[ct] = c < n_cols ? c : n_cols - 1;
    }
    tf_f32x4 acc[2][2];
    for (int ct = 0; ct < 2; ct++)
        for (int tt = 0; tt < 2; tt++) acc[ct][tt] = tf_f32x4{0.f, 0.f, 0.f, 0.f};

    const int xt = tid >> 3, xs = tid & 7;  // staging: token xt, sub-block xs
    const bool xlive = t0 + xt < n_tok;
    const float* xrow = x + (size_t)(xlive ? t0 + xt : 0) * n_rows + 32 * xs;
    const int hc = c0 + tid < n_cols ? c0 + tid : n_cols - 1;
    const uint8_t* hcol = w + (size_t)hc * col_bytes;
    auto load_x = [&](int sb, float4 (&xr)[8]) {
#pragma unroll
        for (int k = 0; k < 8; k++) xr[k] = *reinterpret_cast<const float4*>(xrow + sb * 256 + 4 * k);
    };
    auto load_hdr = [&](int sb, tf_u32x4& hd) {
        if (tid >= TF_PF_COLS) return;
        hd = tf_ld16_a4(hcol + (size_t)sb * 144);
    };
    auto store_x = [&](const float4 (&xr)[8]) {
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 q = xlive ? xr[k] : make_float4(0.f, 0.f, 0.f, 0.f);
            v[4 * k] = q.x;
            v[4 * k + 1] = q.y;
            v[4 * k + 2] = q.z;
            v[4 * k + 3] = q.w;
        }
        float gs = 0.f, amax = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            gs += (v[4 * k] + v[4 * k + 1]) + (v[4 * k + 2] + v[4 * k + 3]);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[4 * k]), fabsf(v[4 * k + 1])),
                                     fmaxf(fabsf(v[4 * k + 2]), fabsf(v[4 * k + 3]))));
        }
        // max over the token's 8 staging threads (consecutive lanes)
        amax = fmaxf(amax, __shfl_xor(amax, 1));
        amax = fmaxf(amax, __shfl_xor(amax, 2));
        amax = fmaxf(amax, __shfl_xor(amax, 4));
        // f = 2^fe with fe = 14 - floor(log2 amax); fe <= 126 keeps 2^-fe a
        // normal float (amax below 2^-112 then scales to below 2^14)
        const int eb = (int)((__float_as_uint(amax) >> 23) & 0xff);
        int fe = amax > 0.f ? 141 - eb : 0;
        fe = fe > 126 ? 126 : fe;
        const float f = __uint_as_float((uint32_t)(fe + 127) << 23);
        if (xs == 0) xinv[xt] = __uint_as_float((uint32_t)(127 - fe) << 23);
        const int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
#pragma unroll
        for (int gg = 0; gg < 4; gg++) {
            uint32_t h0[4], h1[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float a = v[8 * gg + perm[2 * i]] * f, b = v[8 * gg + perm[2 * i + 1]] * f;
                const _Float16 ah = (_Float16)a, bh = (_Float16)b;
                h0[i] = __builtin_bit_cast(uint32_t, tf_h2{ah, bh});
                h1[i] = tf_ph_pk(a - (float)ah, b - (float)bh);
            }
            *reinterpret_cast<tf_u32x4*>(xp + xt * TF_PH_ROW + 2 * (32 * xs + 8 * gg)) =
                tf_u32x4{h0[0], h0[1], h0[2], h0[3]};
            *reinterpret_cast<tf_u32x4*>(xp + (TF_PF_TOKS + xt) * TF_PH_ROW +
                                         2 * (32 * xs + 8 * gg)) =
                tf_u32x4{h1[0], h1[1], h1[2], h1[3]};
        }
        const float sv = gs * f * 0.03125f;  // |sv| <= 2^15
        const _Float16 s0 = (_Float16)sv;
        xsm[xt * 8 + xs] = s0;
        xsm[(TF_PF_TOKS + xt) * 8 + xs] = (_Float16)(sv - (float)s0);
    };
    auto store_hdr = [&](const tf_u32x4& hd) {
        if (tid >= TF_PF_COLS) return;
        dd[tid] = tf_h2f(hd.x);
        dm[tid] = tf_h2f(hd.x >> 16);
        uint8_t s12[12];
        const uint32_t hw[3] = {hd.y, hd.z, hd.w};
#pragma unroll
        for (int i = 0; i < 12; i++) s12[i] = (uint8_t)(hw[i / 4] >> (8 * (i % 4)));
        _Float16 mv[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            int sc, m;
            tf_pf_scale_min(s12, s, sc, m);
            const float scf = (float)sc;
            scn[s * TF_PF_COLS + tid] = make_uint2(tf_ph_pk(scf, scf),
                                                   tf_ph_pk(-1024.f * scf, -1024.f * scf));
            mv[s] = (_Float16)m;
        }
        *reinterpret_cast<tf_h8*>(mh + 8 * tid) =
            tf_h8{mv[0], mv[1], mv[2], mv[3], mv[4], mv[5], mv[6], mv[7]};
    };

    TfPfCol<false> wc[2], wn[2];
    float4 xr[8];
    tf_u32x4 hd = {0, 0, 0, 0};
    uint32_t mask_v = 0x000F000Fu;
    asm volatile("" : "+v"(mask_v));  // keep the mask in a VGPR
    for (int ct = 0; ct < 2; ct++)
        tf_pf_load_col<false>(w + (size_t)colA[ct] * col_bytes + (size_t)sb_lo * 144, g, wc[ct]);
    load_x(sb_lo, xr);
    load_hdr(sb_lo, hd);
    __builtin_amdgcn_s_waitcnt(TF_VMCNT0);  // nothing pending at loop entry (as above)
    for (int sb = sb_lo; sb < sb_hi; sb++) {
        __syncthreads();  // the previous super-block's LDS reads are done
        store_x(xr);
        store_hdr(hd);
        __syncthreads();
        if (sb + 1 < sb_hi) {  // workgroup-uniform
            for (int ct = 0; ct < 2; ct++)
                tf_pf_load_col<false>(w + (size_t)colA[ct] * col_bytes + (size_t)(sb + 1) * 144,
                                      g, wn[ct]);
            load_x(sb + 1, xr);
            load_hdr(sb + 1, hd);
        }
        tf_f32x4 P[2][2], M[2][2];
        for (int ct = 0; ct < 2; ct++)
            for (int tt = 0; tt < 2; tt++) {
                P[ct][tt] = tf_f32x4{0.f, 0.f, 0.f, 0.f};
                M[ct][tt] = tf_f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            tf_h8 b[2][2];
            for (int tt = 0; tt < 2; tt++)
                for (int pl = 0; pl < 2; pl++)
                    b[tt][pl] = *reinterpret_cast<const tf_h8*>(
                        xp + (pl * TF_PF_TOKS + 16 * tt + l16) * TF_PH_ROW + 2 * (32 * s + 8 * g));
            for (int ct = 0; ct < 2; ct++) {
                const uint2 sn = scn[s * TF_PF_COLS + 32 * wave + 16 * ct + l16];
                const tf_h8 a = tf_ph_a(wc[ct].w[2 * (s >> 1)], wc[ct].w[2 * (s >> 1) + 1],
                                        4 * (s & 1), sn, mask_v);
                for (int tt = 0; tt < 2; tt++) {
                    P[ct][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[tt][0], P[ct][tt], 0, 0, 0);
                    P[ct][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[tt][1], P[ct][tt], 0, 0, 0);
                }
            }
        }
        // min term: K = the 8 sub-blocks (lanes g < 2), zero-padded to 16
        {
            tf_h4v bm[2][2], am[2];
            const tf_h4v z = {0, 0, 0, 0};
            for (int tt = 0; tt < 2; tt++)
                for (int pl = 0; pl < 2; pl++)
                    bm[tt][pl] = g < 2 ? *reinterpret_cast<const tf_h4v*>(
                                             xsm + (pl * TF_PF_TOKS + 16 * tt + l16) * 8 + 4 * g)
                                       : z;
            for (int ct = 0; ct < 2; ct++)
                am[ct] = g < 2 ? *reinterpret_cast<const tf_h4v*>(
                                     mh + 8 * (32 * wave + 16 * ct + l16) + 4 * g)
                               : z;
            for (int ct = 0; ct < 2; ct++)
                for (int tt = 0; tt < 2; tt++) {
                    M[ct][tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(am[ct], bm[tt][0], M[ct][tt], 0, 0, 0);
                    M[ct][tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(am[ct], bm[tt][1], M[ct][tt], 0, 0, 0);
                }
        }
        // acc += d 2^-e P - dmin 2^(5-e) M; C rows 4g+r = columns, C column l16 = token
        for (int ct = 0; ct < 2; ct++) {
            const int cl = 32 * wave + 16 * ct + 4 * g;
            const float4 d4 = *reinterpret_cast<const float4*>(dd + cl);
            const float4 m4 = *reinterpret_cast<const float4*>(dm + cl);
            const float dv[4] = {d4.x, d4.y, d4.z, d4.w}, mv[4] = {m4.x, m4.y, m4.z, m4.w};
            for (int tt = 0; tt < 2; tt++) {
                const float fi = xinv[16 * tt + l16];
                for (int r = 0; r < 4; r++) {
                    float v = acc[ct][tt][r] + (dv[r] * fi) * P[ct][tt][r];
                    acc[ct][tt][r] = v - (mv[r] * (32.f * fi)) * M[ct][tt][r];
                }
            }
        }
        for (int ct = 0; ct < 2; ct++) wc[ct] = wn[ct];
    }
    for (int ct = 0; ct < 2; ct++) {
        const int cb = c0 + 32 * wave + 16 * ct + 4 * g;
        for (int tt = 0; tt < 2; tt++) {
            const int t = t0 + 16 * tt + l16;
            if (t >= n_tok) continue;
            float* o = out + (size_t)t * n_cols + cb;
            if (cb + 3 < n_cols && ((n_cols & 3) == 0)) {
                float4 v = make_float4(acc[ct][tt][0], acc[ct][tt][1], acc[ct][tt][2],
                                       acc[ct][tt][3]);
                if (accumulate) {
                    const float4 o0 = *reinterpret_cast<const float4*>(o);
                    v = make_float4(o0.x + v.x, o0.y + v.y, o0.z + v.z, o0.w + v.w);
                }
                *reinterpret_cast<float4*>(o) = v;
            } else {
                for (int r = 0; r < 4; r++)
                    if (cb + r < n_cols) o[r] = accumulate ? o[r] + acc[ct][tt][r] : acc[ct][tt][r];
            }
        }
    }
}

// ---------------------------------------------------------------- attention
//
// Causal attention of n_q queries (positions pos0 .. pos0+n_q-1) over the
// f16 cache, fp32 arithmetic.  A workgroup (256 threads) owns one head and
// 16 consecutive queries; K/V tiles of T keys (64, 32, 16 for head_dim 64,
// 128, 256: about 45 KB of LDS) are staged in LDS as f32 and shared by the
// 16 queries.  Thread (query qi = tid / 16, m = tid % 16): scores of keys
// m, m+16, ... of the tile (a DPP row holds one query, so the row max and
// sum are row reductions), then output dims DPT m .. DPT m + DPT-1 with
// DPT = head_dim / 16.  Online softmax as
// the reference: m_new = max(m, tile max), alpha = e^(m - m_new),
// l = l alpha + tile sum, out = acc / max(l, 1e-20).

#define TF_PA_Q 16

template <int HD>
__global__ __launch_bounds__(256) void tf_attn_prefill_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    float* __restrict__ out, int n_head, int n_kv, int pos0_arg, const int* __restrict__ pos0_ptr,
    int n_q, float scale) {
    constexpr int DPT = HD / 16;  // output dims per thread
    constexpr int TF_PA_T = HD == 64 ? 64 : (HD == 128 ? 32 : 16);  // keys per tile
    constexpr int NS = TF_PA_T / 16;                                // scores per thread
    __shared__ __align__(16) float qs[TF_PA_Q * (HD + 4)];
    __shared__ __align__(16) float ks[TF_PA_T * (HD + 4)];
    __shared__ __align__(16) float vs[TF_PA_T * HD];
    __shared__ float ps[TF_PA_Q * (TF_PA_T + 1)];
    const int pos0 = pos0_ptr ? pos0_ptr[0] : pos0_arg;
    const int h = blockIdx.y, q0 = blockIdx.x * TF_PA_Q;
    const int tid = threadIdx.x, qi = tid >> 4, m = tid & 15;
    const int kv_h = h / (n_head / n_kv), stride = n_kv * HD;
    const int qn = q0 + qi;
    const bool qvalid = qn < n_q;
    const int my_len = pos0 + (qvalid ? qn : q0) + 1;           // keys this query sees
    const int last_q = (q0 + TF_PA_Q < n_q ? q0 + TF_PA_Q : n_q) - 1;
    const int seq_len = pos0 + last_q + 1;                         // keys of the workgroup
    for (int i = tid; i < TF_PA_Q * HD / 4; i += 256) {
        const int r = i / (HD / 4), c4 = i % (HD / 4);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (q0 + r < n_q)
            v = *reinterpret_cast<const float4*>(q + (size_t)(q0 + r) * n_head * HD + h * HD + 4 * c4);
        *reinterpret_cast<float4*>(qs + r * (HD + 4) + 4 * c4) = v;
    }
    float mx = -1e30f, l = 0.f, acc[DPT];
    for (int i = 0; i < DPT; i++) acc[i] = 0.f;
    for (int t0 = 0; t0 < seq_len; t0 += TF_PA_T) {
        const int tlen = seq_len - t0 < TF_PA_T ? seq_len - t0 : TF_PA_T;
        __syncthreads();  // q staged / previous tile consumed
        for (int i = tid; i < TF_PA_T * HD / 4; i += 256) {
            const int r = i / (HD / 4), c4 = i % (HD / 4);
            float4 kf = make_float4(0.f, 0.f, 0.f, 0.f), vf = kf;
            if (r < tlen) {
                const size_t off = (size_t)(t0 + r) * stride + (size_t)kv_h * HD + 4 * c4;
                const uint2 kb = *reinterpret_cast<const uint2*>(kc + off);
                const uint2 vb = *reinterpret_cast<const uint2*>(vc + off);
                kf = make_float4(tf_h2f(kb.x), tf_h2f(kb.x >> 16), tf_h2f(kb.y), tf_h2f(kb.y >> 16));
                vf = make_float4(tf_h2f(vb.x), tf_h2f(vb.x >> 16), tf_h2f(vb.y), tf_h2f(vb.y >> 16));
            }
            *reinterpret_cast<float4*>(ks + r * (HD + 4) + 4 * c4) = kf;
            *reinterpret_cast<float4*>(vs + r * HD + 4 * c4) = vf;
        }
        __syncthreads();
        // scores of keys m + 16 j
        float s[NS];
        const float* qrow = qs + qi * (HD + 4);
#pragma unroll
        for (int j = 0; j < NS; j++) {
            const float* krow = ks + (m + 16 * j) * (HD + 4);
            float a0 = 0.f, a1 = 0.f;
            for (int d = 0; d < HD; d += 8) {
                const float4 qa = *reinterpret_cast<const float4*>(qrow + d);
                const float4 qb = *reinterpret_cast<const float4*>(qrow + d + 4);
                const float4 ka = *reinterpret_cast<const float4*>(krow + d);
                const float4 kb = *reinterpret_cast<const float4*>(krow + d + 4);
                a0 += qa.x * ka.x + qa.y * ka.y + qa.z * ka.z + qa.w * ka.w;
                a1 += qb.x * kb.x + qb.y * kb.y + qb.z * kb.z + qb.w * kb.w;
            }
            const int key = t0 + m + 16 * j;
            s[j] = key < my_len ? (a0 + a1) * scale : -1e30f;
        }
        float tmax = s[0];
#pragma unroll
        for (int j = 1; j < NS; j++) tmax = fmaxf(tmax, s[j]);
        tmax = tf_row16_max(tmax);
        const float m_new = fmaxf(mx, tmax);
        const float alpha = __expf(mx - m_new);
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < NS; j++) {
            const float e = s[j] > -1e29f ? __expf(s[j] - m_new) : 0.f;
            ps[qi * (TF_PA_T + 1) + m + 16 * j] = e;
            ls += e;
        }
        ls = tf_row16_sum(ls);
        l = l * alpha + ls;
        mx = m_new;
        for (int i = 0; i < DPT; i++) acc[i] *= alpha;
        __syncthreads();  // ps complete (the row's other lanes wrote it)
        const float* prow = ps + qi * (TF_PA_T + 1);
        for (int t = 0; t < tlen; t++) {
            const float p = prow[t];
            const float* vrow = vs + t * HD + DPT * m;
#pragma unroll
            for (int i = 0; i < DPT; i += 4) {
                const float4 v = *reinterpret_cast<const float4*>(vrow + i);
                acc[i] += p * v.x;
                acc[i + 1] += p * v.y;
                acc[i + 2] += p * v.z;
                acc[i + 3] += p * v.w;
            }
        }
    }
    if (qvalid) {
        const float inv = 1.f / fmaxf(l, 1e-20f);
        float* o = out + (size_t)qn * n_head * HD + h * HD + DPT * m;
        for (int i = 0; i < DPT; i += 4)
            *reinterpret_cast<float4*>(o + i) =
                make_float4(acc[i] * inv, acc[i + 1] * inv, acc[i + 2] * inv, acc[i + 3] * inv);
    }
}

// Matrix-core form for head_dim 128.  A workgroup (4 waves) owns one head
// and 16 queries; the waves split the 32-key tiles round-robin, each staging
// its own tiles in LDS, and merge their (m, l, O) with the log-sum-exp rule
// at the end (a wave with no keys for a query contributes e^(-1e30 - M) = 0).
// Per tile, on v_mfma_f32_16x16x32_f16:
//   S^T = K q^T: A = K rows (A row i of key block b is key
//       8 (i / 4) + 4 b + i % 4, so the C values a lane holds, key rows
//       4g .. 4g+3 of blocks 0 and 1, are the tile's keys 8g .. 8g+7), B =
//       q^T, q split into two f16 parts after a power-of-two scale (2^-22
//       relative per product; K is f16, the products are exact);
//   O += P V: A = P (query l16, keys 8g .. 8g+7: the lane's own S values
//       after the softmax, split into two f16 parts), B = V gathered from
//       the row-major f16 tile (8 u16 reads per fragment).
// Softmax per query: the lane's 8 values, then the 4 lanes of the query
// (xor 16, 32).  Keys past the workgroup's last query are staged as zeros.

#define TF_PM_T 32              // keys per tile
#define TF_PM_KROW 272          // K tile row bytes (128 f16 + 16)
#define TF_PM_VROW 264          // V tile row bytes (128 f16 + 8): 8-row gathers on distinct banks
#define TF_PM_WAVE_BYTES (TF_PM_T * TF_PM_KROW + TF_PM_T * TF_PM_VROW)

__global__ __launch_bounds__(256) void tf_attn_prefill_mfma_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    float* __restrict__ out, int n_head, int n_kv, int pos0_arg, const int* __restrict__ pos0_ptr,
    int n_q, float scale) {
    constexpr int HD = 128;
    __shared__ __align__(16) uint8_t lds[4 * TF_PM_WAVE_BYTES];
    __shared__ float ml[2][4][16];
    const int pos0 = pos0_ptr ? pos0_ptr[0] : pos0_arg;
    const int h = blockIdx.y, q0 = blockIdx.x * 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int kv_h = h / (n_head / n_kv), stride = n_kv * HD;
    const int last_q = (q0 + 16 < n_q ? q0 + 16 : n_q) - 1;
    const int kv_len = pos0 + last_q + 1;  // keys the workgroup reads
    const int n_t = (kv_len + TF_PM_T - 1) / TF_PM_T;
    uint8_t* kt = lds + wave * TF_PM_WAVE_BYTES;
    uint8_t* vt = kt + TF_PM_T * TF_PM_KROW;

    // q^T fragments: query l16, dims 32 st + 8 g .. +7, two f16 parts
    const int my_q = q0 + l16 < n_q ? q0 + l16 : last_q;
    const int qpos = pos0 + my_q;
    float qv[32];
    {
        const float* qr = q + (size_t)my_q * n_head * HD + (size_t)h * HD;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const float4 a = *reinterpret_cast<const float4*>(qr + 32 * st + 8 * g);
            const float4 b = *reinterpret_cast<const float4*>(qr + 32 * st + 8 * g + 4);
            qv[8 * st] = a.x; qv[8 * st + 1] = a.y; qv[8 * st + 2] = a.z; qv[8 * st + 3] = a.w;
            qv[8 * st + 4] = b.x; qv[8 * st + 5] = b.y; qv[8 * st + 6] = b.z; qv[8 * st + 7] = b.w;
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(qv[i]));
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const int eb = (int)((__float_as_uint(amax) >> 23) & 0xff);
    int fe = amax > 0.f ? 141 - eb : 0;
    fe = fe > 126 ? 126 : fe;
    const float f = __uint_as_float((uint32_t)(fe + 127) << 23);
    const float sscale = scale * __uint_as_float((uint32_t)(127 - fe) << 23);
    tf_h8 qb[4][2];
#pragma unroll
    for (int st = 0; st < 4; st++)
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float a = qv[8 * st + i] * f;
            const _Float16 hi = (_Float16)a;
            qb[st][0][i] = hi;
            qb[st][1][i] = (_Float16)(a - (float)hi);
        }

    float mx = -1e30f, l = 0.f;
    tf_f32x4 o[8];
#pragma unroll
    for (int nb = 0; nb < 8; nb++) o[nb] = tf_f32x4{0.f, 0.f, 0.f, 0.f};

    for (int ti = wave; ti < n_t; ti += 4) {
        const int t0 = ti * TF_PM_T;
        // stage K and V rows t0 .. t0+31 (zeros past kv_len)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int idx = lane + 64 * j, r = idx >> 4, c = idx & 15;
            tf_u32x4 kb = {0, 0, 0, 0}, vb = {0, 0, 0, 0};
            if (t0 + r < kv_len) {
                const size_t off = (size_t)(t0 + r) * stride + (size_t)kv_h * HD + 8 * c;
                kb = *reinterpret_cast<const tf_u32x4*>(kc + off);
                vb = *reinterpret_cast<const tf_u32x4*>(vc + off);
            }
            *reinterpret_cast<tf_u32x4*>(kt + r * TF_PM_KROW + 16 * c) = kb;
            uint32_t* vw = reinterpret_cast<uint32_t*>(vt + r * TF_PM_VROW + 16 * c);
            vw[0] = vb.x; vw[1] = vb.y; vw[2] = vb.z; vw[3] = vb.w;  // 8-byte aligned rows
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_s_waitcnt(0xc07f);  // LDS stores of the wave done (lgkmcnt 0)
        __builtin_amdgcn_wave_barrier();
        // S^T: two key blocks, 4 K steps, 2 parts
        tf_f32x4 sc[2];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int key = 8 * (l16 >> 2) + 4 * b + (l16 & 3);
            tf_f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; st++) {
                const tf_h8 ka = *reinterpret_cast<const tf_h8*>(kt + key * TF_PM_KROW +
                                                                 2 * (32 * st + 8 * g));
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[st][0], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[st][1], c, 0, 0, 0);
            }
            sc[b] = c;
        }
        // lane values: keys t0 + 8g + 4b + r of query my_q
        float sv[8];
        float tmax = -1e30f;
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int kp = t0 + 8 * g + 4 * b + r;
                const float v = kp <= qpos ? sc[b][r] * sscale : -1e30f;
                sv[4 * b + r] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(mx, tmax);
        const float alpha = __expf(mx - m_new);
        float ls = 0.f;
        tf_h8 pa[2];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float e = sv[i] > -1e29f ? __expf(sv[i] - m_new) : 0.f;
            ls += e;
            const _Float16 hi = (_Float16)e;
            pa[0][i] = hi;
            pa[1][i] = (_Float16)(e - (float)hi);
        }
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        l = l * alpha + ls;
        mx = m_new;
        // O rows are queries 4g .. 4g+3: their alpha from lanes 4g + r
        float al[4];
#pragma unroll
        for (int r = 0; r < 4; r++) al[r] = __shfl(alpha, 4 * g + r);
#pragma unroll
        for (int nb = 0; nb < 8; nb++) {
#pragma unroll
            for (int r = 0; r < 4; r++) o[nb][r] *= al[r];
            // V fragment: keys 8g .. 8g+7, dim 16 nb + l16
            const uint8_t* vp = vt + (8 * g) * TF_PM_VROW + 2 * (16 * nb + l16);
            tf_h8 vf;
#pragma unroll
            for (int i = 0; i < 8; i++)
                vf[i] = __builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(vp + i * TF_PM_VROW));
            o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[0], vf, o[nb], 0, 0, 0);
            o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[1], vf, o[nb], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();  // tile reads done before the next staging
    }
    // merge the 4 waves: (m, l) per query, O through LDS
    if (g == 0) {
        ml[0][wave][l16] = mx;
        ml[1][wave][l16] = l;
    }
    __syncthreads();  // every wave's tiles consumed; ml visible
    float* ow = reinterpret_cast<float*>(lds + wave * TF_PM_WAVE_BYTES);  // [16][128]
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int qi = 4 * g + r;
        float mall = ml[0][0][qi];
        for (int w = 1; w < 4; w++) mall = fmaxf(mall, ml[0][w][qi]);
        const float sc_w = __expf(ml[0][wave][qi] - mall);
#pragma unroll
        for (int nb = 0; nb < 8; nb++) ow[qi * HD + 16 * nb + l16] = o[nb][r] * sc_w;
    }
    __syncthreads();
    {
        const int qi = tid >> 4, d0 = 8 * (tid & 15);
        if (q0 + qi < n_q) {
            float mall = ml[0][0][qi];
            for (int w = 1; w < 4; w++) mall = fmaxf(mall, ml[0][w][qi]);
            float L = 0.f;
            for (int w = 0; w < 4; w++) L += ml[1][w][qi] * __expf(ml[0][w][qi] - mall);
            const float inv = 1.f / fmaxf(L, 1e-20f);
            float acc[8];
            for (int i = 0; i < 8; i++) acc[i] = 0.f;
            for (int w = 0; w < 4; w++) {
                const float* src = reinterpret_cast<const float*>(lds + w * TF_PM_WAVE_BYTES) + qi * HD + d0;
                for (int i = 0; i < 8; i++) acc[i] += src[i];
            }
            float* dst = out + (size_t)(q0 + qi) * n_head * HD + (size_t)h * HD + d0;
            *reinterpret_cast<float4*>(dst) = make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
            *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv);
        }
    }
}

// ------------------------------------------------- batched prefill glue
//
// The n_tok-row forms of the decode glue (kernels/ops.cu rms_norm_f32 with
// n_tok rows :4-34, add_bias_f32 :340, rope_neox_f32 :348, copy_kv_f16
// :471, silu_mul_f32 :202; kernels/embed.cu embed_q{4,6}_k :1-50), used by
// the runtime's prefill step.

template <int BB>
__global__ __launch_bounds__(256) void tf_pf_embed_kernel(const uint8_t* __restrict__ table,
                                                          const int* __restrict__ tokens,
                                                          float* __restrict__ out, int n_rows,
                                                          int col_bytes) {
    const int t = blockIdx.y;
    const uint8_t* col = table + (size_t)tokens[t] * col_bytes;
    const int nb = n_rows / 256;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nb * 256; i += gridDim.x * blockDim.x) {
        const uint8_t* blk = col + (size_t)(i >> 8) * BB;
        out[(size_t)t * n_rows + i] = BB == 144 ? tf_q4k_value(blk, i & 255) : tf_q6k_value(blk, i & 255);
    }
}

// One row per workgroup, the decode RMSNorm's order (256 strided fused
// square sums, halving tree).
__global__ __launch_bounds__(256) void tf_pf_rms_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ w,
                                                        float* __restrict__ out, int n, float eps) {
    __shared__ float buf[256];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* orow = out + (size_t)blockIdx.x * n;
    float local = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i];
        local = fmaf(v, v, local);
    }
    buf[threadIdx.x] = local;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) buf[threadIdx.x] += buf[threadIdx.x + s];
        __syncthreads();
    }
    const float scale = 1.0f / sqrtf(buf[0] / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) orow[i] = xr[i] * scale * w[i];
}

// q/k/v rows of token t (position pos0 + t): add the biases, rotate q and k
// (NeoX pairs (i, i + hd/2) by (pos0+t) theta^(-2i/hd)), append k and v to
// the f16 cache.  Grid (n_head + 2 n_kv, n_tok): head blocks of q, then k,
// then v.
__global__ __launch_bounds__(64) void tf_pf_qkv_post_kernel(
    float* __restrict__ q, float* __restrict__ k, float* __restrict__ v,
    const float* __restrict__ bq, const float* __restrict__ bk, const float* __restrict__ bv,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int n_head, int n_kv, int hd, int pos0,
    float theta) {
    const int t = blockIdx.y, hb = blockIdx.x;
    const int kvd = n_kv * hd, pos = pos0 + t;
    float* base;
    const float* b;
    uint16_t* cache = nullptr;
    bool rot = true;
    if (hb < n_head) {
        base = q + (size_t)t * n_head * hd + hb * hd;
        b = bq ? bq + hb * hd : nullptr;
    } else if (hb < n_head + n_kv) {
        const int h = hb - n_head;
        base = k + (size_t)t * kvd + h * hd;
        b = bk ? bk + h * hd : nullptr;
        cache = kc + (size_t)pos * kvd + h * hd;
    } else {
        const int h = hb - n_head - n_kv;
        base = v + (size_t)t * kvd + h * hd;
        b = bv ? bv + h * hd : nullptr;
        cache = vc + (size_t)pos * kvd + h * hd;
        rot = false;
    }
    const int half = hd / 2;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        float x0 = base[i], x1 = base[i + half];
        if (b) {
            x0 += b[i];
            x1 += b[i + half];
        }
        if (rot) {
            const float freq = powf(theta, -2.f * (float)i / (float)hd);
            const float ang = (float)pos * freq;
            float sn, cs;
            sincosf(ang, &sn, &cs);
            const float r0 = x0 * cs - x1 * sn, r1 = x0 * sn + x1 * cs;
            x0 = r0;
            x1 = r1;
        }
        base[i] = x0;
        base[i + half] = x1;
        if (cache) {
            cache[i] = tf_f2h_halfup(x0);
            cache[i + half] = tf_f2h_halfup(x1);
        }
    }
}

__global__ __launch_bounds__(256) void tf_pf_silu_mul_kernel(float* __restrict__ g,
                                                             const float* __restrict__ u,
                                                             long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = g[i];
        g[i] = (v / (1.f + __expf(-v))) * u[i];
    }
}

int tf_pf_embed(const uint8_t* table, int block_bytes, const int* tokens_dev, float* out,
                int n_rows, int col_bytes, int n_tok, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(table && tokens_dev && out && nb > 0 && n_tok > 0);
    TF_CHECK_ARG((block_bytes == 144 || block_bytes == 210) && col_bytes >= nb * block_bytes);
    const dim3 grid((nb * 256 + 255) / 256, n_tok);
    if (block_bytes == 144)
        hipLaunchKernelGGL(tf_pf_embed_kernel<144>, grid, dim3(256), 0, tf_stream(stream), table,
                           tokens_dev, out, n_rows, col_bytes);
    else
        hipLaunchKernelGGL(tf_pf_embed_kernel<210>, grid, dim3(256), 0, tf_stream(stream), table,
                           tokens_dev, out, n_rows, col_bytes);
    return TF_LAUNCH_RESULT();
}

int tf_pf_rms_norm(const float* x, const float* w, float* out, int n, int n_tok, float eps,
                   tf_stream_t stream) {
    TF_CHECK_ARG(x && w && out && n > 0 && n_tok > 0);
    hipLaunchKernelGGL(tf_pf_rms_kernel, dim3(n_tok), dim3(256), 0, tf_stream(stream), x, w, out,
                       n, eps);
    return TF_LAUNCH_RESULT();
}

int tf_pf_qkv_post(float* q, float* k, float* v, const float* bq, const float* bk,
                   const float* bv, uint16_t* k_cache, uint16_t* v_cache, int n_head, int n_kv,
                   int head_dim, int pos0, int n_tok, float theta, tf_stream_t stream) {
    TF_CHECK_ARG(q && k && v && k_cache && v_cache && n_head > 0 && n_kv > 0 && n_tok > 0);
    TF_CHECK_ARG(head_dim > 0 && (head_dim & 1) == 0 && pos0 >= 0);
    hipLaunchKernelGGL(tf_pf_qkv_post_kernel, dim3(n_head + 2 * n_kv, n_tok), dim3(64), 0,
                       tf_stream(stream), q, k, v, bq, bk, bv, k_cache, v_cache, n_head, n_kv,
                       head_dim, pos0, theta);
    return TF_LAUNCH_RESULT();
}

int tf_pf_silu_mul(float* g, const float* u, long long n, tf_stream_t stream) {
    TF_CHECK_ARG(g && u && n > 0);
    hipLaunchKernelGGL(tf_pf_silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       tf_stream(stream), g, u, n);
    return TF_LAUNCH_RESULT();
}

// out[i] (+)= sum over z of part[z][i], z in order (split-K of the GEMM).
__global__ __launch_bounds__(256) void tf_gemm_split_reduce_kernel(const float* __restrict__ part,
                                                                   float* __restrict__ out,
                                                                   long long n4, int n_split,
                                                                   int accumulate) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4* p = reinterpret_cast<const float4*>(part) + i;
    float4 v = p[0];
    for (int z = 1; z < n_split; z++) {
        const float4 q = p[(size_t)z * (size_t)n4];
        v = make_float4(v.x + q.x, v.y + q.y, v.z + q.z, v.w + q.w);
    }
    float4* o = reinterpret_cast<float4*>(out) + i;
    if (accumulate) {
        const float4 r = *o;
        v = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
    }
    *o = v;
}

// ---------------------------------------------------------------- C ABI

int tf_gemm_kq(bool q6, const uint8_t* w, const float* x, float* out, int n_rows, int n_cols,
               int col_bytes, int n_tok, int accumulate, tf_stream_t stream, float* ws,
               size_t ws_floats) {
    const int nb = n_rows / 256;
    const int blk = q6 ? 210 : 144;
    TF_CHECK_ARG(w && x && out && nb > 0 && n_cols > 0 && n_tok > 0);
    // nb = n_rows / 256 floors a partial last super-block away, as the
    // reference's gemm_q4_k / gemm_q6_k do (kernels/gemm.cu:28, :89); the
    // GPU tests pin that case (K = 896 -> three super-blocks)
    TF_CHECK_ARG(col_bytes >= nb * blk && (n_rows & 3) == 0 && ((uintptr_t)x & 15) == 0);
    if (q6) TF_CHECK_ARG(((uintptr_t)w & 1) == 0 && (col_bytes & 1) == 0);
    else TF_CHECK_ARG(((uintptr_t)w & 3) == 0 && (col_bytes & 3) == 0);
    TF_CHECK_ARG(((uintptr_t)out & 15) == 0);
    const size_t tiles = (size_t)((n_tok + TF_PF_TOKS - 1) / TF_PF_TOKS) *
                         ((n_cols + TF_PF_COLS - 1) / TF_PF_COLS);
    TF_CHECK_ARG(tiles <= (size_t)1 << 28);
    // one-dimensional grid, 8 x ceil(tiles / 8) workgroups (the kernel maps
    // them XCD by XCD; the padding exits at once)
    dim3 grid((unsigned)(8 * ((tiles + 7) / 8)), 1);
    // Split-K when the tile grid leaves the chip short of workgroups: about
    // 512 workgroups in all (measured on the 3B prefill against 384, 768, 1024
    // and 1536), partial slices into ws, then a fixed-order sum.
    const size_t slice = (size_t)n_tok * n_cols;
    int n_split = 1;
    if (ws && tiles < 384 && (n_cols & 3) == 0 && ((uintptr_t)ws & 15) == 0) {
        constexpr int target = 512;
        n_split = (int)((target + tiles - 1) / tiles);
        if (n_split > nb) n_split = nb;
        while (n_split > 1 && (size_t)n_split * slice > ws_floats) n_split--;
    }
    grid.z = n_split;
    float* dst = n_split > 1 ? ws : out;
    const int acc = n_split > 1 ? 0 : accumulate;
    if (q6)
        hipLaunchKernelGGL(tf_gemm_kq_kernel<true>, grid, dim3(256), 0, tf_stream(stream), w, x,
                           dst, n_rows, n_cols, col_bytes, n_tok, acc, n_split, (long long)slice);
    else
        hipLaunchKernelGGL(tf_gemm_q4k_h_kernel, grid, dim3(256), 0, tf_stream(stream), w, x,
                           dst, n_rows, n_cols, col_bytes, n_tok, acc, n_split, (long long)slice);
    if (n_split > 1) {
        const long long n4 = (long long)(slice / 4);
        hipLaunchKernelGGL(tf_gemm_split_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)),
                           dim3(256), 0, tf_stream(stream), ws, out, n4, n_split, accumulate);
    }
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_gemm_q4k_f32(const uint8_t* w, const float* x, float* out, int n_rows,
                               int n_cols, int col_bytes, int n_tok, tf_stream_t stream) {
    return tf_gemm_kq(false, w, x, out, n_rows, n_cols, col_bytes, n_tok, 0, stream, nullptr, 0);
}

extern "C" int tf_gemm_q6k_f32(const uint8_t* w, const float* x, float* out, int n_rows,
                               int n_cols, int col_bytes, int n_tok, tf_stream_t stream) {
    return tf_gemm_kq(true, w, x, out, n_rows, n_cols, col_bytes, n_tok, 0, stream, nullptr, 0);
}

int tf_attn_prefill_any(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                               float* out, int n_head, int n_kv, int head_dim, int pos0,
                               const int* pos0_dev, int n_q, float scale, tf_stream_t stream) {
    TF_CHECK_ARG(q && k_cache && v_cache && out && n_head > 0 && n_kv > 0 && n_q > 0);
    TF_CHECK_ARG(n_head % n_kv == 0 && (pos0_dev || pos0 >= 0));
    TF_CHECK_ARG(head_dim == 64 || head_dim == 128 || head_dim == 256);
    TF_CHECK_ARG(((uintptr_t)q & 15) == 0 && ((uintptr_t)out & 15) == 0);
    TF_CHECK_ARG(((uintptr_t)k_cache & 7) == 0 && ((uintptr_t)v_cache & 7) == 0);
    const dim3 grid((n_q + TF_PA_Q - 1) / TF_PA_Q, n_head);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, tf_stream(stream), q, k_cache, v_cache, out,
                           n_head, n_kv, pos0, pos0_dev, n_q, scale);
    };
    if (head_dim == 64) go(tf_attn_prefill_kernel<64>);
    else if (head_dim == 128) {
        const dim3 g16((n_q + 15) / 16, n_head);
        hipLaunchKernelGGL(tf_attn_prefill_mfma_kernel, g16, dim3(256), 0, tf_stream(stream), q,
                           k_cache, v_cache, out, n_head, n_kv, pos0, pos0_dev, n_q, scale);
    } else go(tf_attn_prefill_kernel<256>);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_attn_prefill(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                               float* out, int n_head, int n_kv, int head_dim, int pos0, int n_q,
                               float scale, tf_stream_t stream) {
    return tf_attn_prefill_any(q, k_cache, v_cache, out, n_head, n_kv, head_dim, pos0, nullptr,
                               n_q, scale, stream);
}

extern "C" int tf_attn_prefill_d(const float* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, float* out, int n_head, int n_kv,
                                 int head_dim, const int* pos0_dev, int n_q, float scale,
                                 tf_stream_t stream) {
    TF_CHECK_ARG(pos0_dev != nullptr);
    return tf_attn_prefill_any(q, k_cache, v_cache, out, n_head, n_kv, head_dim, 0, pos0_dev, n_q,
                               scale, stream);
}
