/*
 * CPU oracle for the taraference batch-1 decode hot path -- TEST
 * INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).
 *
 * Citations are to agkomyint/taraference v0.5.3, relative to
 * crates/core/src/cuda/.  Build with -ffp-contract=off so that every fp32
 * expression rounds exactly as written (the reference's NVRTC build may fuse
 * multiply-adds; that freedom is absorbed by the tests' tolerances).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- helpers */

/* Exact IEEE binary16 -> binary32 (kernels/common.cu:2-6 uses the hardware
 * cvt.f32.f16, which is exact for every input; cuda/../quant.rs:13-40 is the
 * host twin). */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do {
                mant <<= 1;
                e++;
            } while ((mant & 0x400u) == 0);
            mant &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* kernels/common.cu:9-38 float_to_half_bits: truncate, then add one ulp when
 * the first dropped bit is set (round half up on magnitude, not RNE). */
uint16_t or_f32_to_f16_halfup(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx == 0u) return (uint16_t)sign;
    if (absx >= 0x7f800000u) {
        if (absx == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u);
    }
    if (absx < 0x33000000u) return (uint16_t)sign;
    if (absx >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);
    int e = (int)((absx >> 23) & 0xff) - 127 + 15;
    uint32_t mant = absx & 0x7fffffu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_mant = mant >> shift;
        if ((mant >> (shift - 1)) & 1u) half_mant += 1u;
        return (uint16_t)(sign | half_mant);
    }
    uint32_t half = ((uint32_t)e << 10) | (mant >> 13);
    if (mant & 0x1000u) half += 1u;
    return (uint16_t)(sign | half);
}

static inline uint16_t rd16(const uint8_t *p) {
    return (uint16_t)(p[0] | (p[1] << 8));
}
static inline int32_t rd32(const void *p) {
    int32_t v;
    memcpy(&v, p, 4);
    return v;
}
static inline uint32_t rdu32(const void *p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

/* CUDA __dp4a(int a, int b, int c): four signed byte products plus c. */
static inline int32_t dp4a(int32_t a, int32_t b, int32_t c) {
    int32_t s = c;
    for (int i = 0; i < 4; i++) {
        int8_t ab = (int8_t)((uint32_t)a >> (8 * i));
        int8_t bb = (int8_t)((uint32_t)b >> (8 * i));
        s += (int32_t)ab * (int32_t)bb;
    }
    return s;
}

/* CUDA __vsubss4: per-byte signed saturating a - b. */
static inline int32_t vsubss4(int32_t a, int32_t b) {
    uint32_t r = 0;
    for (int i = 0; i < 4; i++) {
        int v = (int)(int8_t)((uint32_t)a >> (8 * i)) -
                (int)(int8_t)((uint32_t)b >> (8 * i));
        if (v > 127) v = 127;
        if (v < -128) v = -128;
        r |= ((uint32_t)(uint8_t)(int8_t)v) << (8 * i);
    }
    return (int32_t)r;
}

/* kernels/common.cu:52-59 warp_sum: shfl_down tree 16,8,4,2,1; lane 0. */
static float warp_sum32(const float *v) {
    float s[32];
    memcpy(s, v, sizeof(s));
    for (int off = 16; off >= 1; off >>= 1)
        for (int i = 0; i < off; i++) s[i] = s[i] + s[i + off];
    return s[0];
}

/* kernels/common.cu:40-50 get_scale_min_k4 */
static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* ------------------------------------------------------------- Q8 quantize */

/* kernels/gemv.cu:43-65.  One 32-value group per warp: amax by shuffle tree
 * (max is order-free), d = amax * fl(1/127), q = rint_even(x / d) with an
 * IEEE division (the reference's NVRTC fast-math divide is approximate; this
 * restatement fixes IEEE semantics).  n_rows must be a multiple of 32. */
void or_quantize_q8(const float *x, int8_t *q8, float *d8, int n_rows) {
    const int nb = n_rows >> 5;
    const float inv127 = 1.0f / 127.0f;
    for (int bi = 0; bi < nb; bi++) {
        float amax = 0.f;
        for (int l = 0; l < 32; l++) amax = fmaxf(amax, fabsf(x[bi * 32 + l]));
        const float d = amax * inv127;
        for (int l = 0; l < 32; l++) {
            const int i = bi * 32 + l;
            q8[i] = amax == 0.f ? 0 : (int8_t)lrintf(x[i] / d);
        }
        d8[bi] = d;
    }
}

/* --------------------------------------------------------- exact int sums */

void or_q4k_block_dots(const uint8_t *col, const int8_t *q8, int nsb,
                       int32_t *dots, int32_t *sums) {
    for (int bi = 0; bi < nsb; bi++) {
        const uint8_t *qs = col + bi * 144 + 16;
        for (int g = 0; g < 8; g++) {
            const int t = g >> 1, hi = g & 1;
            int32_t dot = 0, sum = 0;
            for (int l = 0; l < 32; l++) {
                const int nib = hi ? (qs[32 * t + l] >> 4) : (qs[32 * t + l] & 0xF);
                const int a = q8[bi * 256 + 32 * g + l];
                dot += nib * a;
                sum += a;
            }
            dots[bi * 8 + g] = dot;
            sums[bi * 8 + g] = sum;
        }
    }
}

/* Q6_K value v of a super-block (kernels/common.cu:164-186 layout). */
static int q6_value(const uint8_t *base, int v) {
    const int n = v >> 7, r = v & 127, k = r >> 5, l = r & 31;
    const uint8_t *ql = base + 64 * n;
    const uint8_t qh = base[128 + 32 * n + l];
    int lo;
    switch (k) {
    case 0: lo = ql[l] & 0xF; break;
    case 1: lo = ql[32 + l] & 0xF; break;
    case 2: lo = ql[l] >> 4; break;
    default: lo = ql[32 + l] >> 4; break;
    }
    return (lo | (((qh >> (2 * k)) & 3) << 4)) - 32;
}

void or_q6k_block_dots(const uint8_t *col, int block_bytes, const int8_t *q8,
                       int nsb, int32_t *dots) {
    for (int bi = 0; bi < nsb; bi++) {
        const uint8_t *base = col + (size_t)bi * block_bytes;
        for (int g = 0; g < 16; g++) {
            int32_t dot = 0;
            for (int i = 0; i < 16; i++) {
                const int v = 16 * g + i;
                dot += q6_value(base, v) * q8[bi * 256 + v];
            }
            dots[bi * 16 + g] = dot;
        }
    }
}

/* ------------------------------------------------------------ Q4_K x Q8 */

/* kernels/gemv.cu:71-130 dot_q4_k_col_q8_range, all 32 lanes, then warp_sum.
 * q8/d8 point at super-block bi0 (local indexing, as the reference). */
static float dot_q4k_warp(const uint8_t *col, const int8_t *q8, const float *d8,
                          int bi0, int bi1) {
    float acc[32];
    for (int lane = 0; lane < 32; lane++) {
        float a = 0.f;
        const int l16 = lane & 15;
        const int q8_offset = 2 * (l16 >> 2);
        const int q4_offset = 16 * q8_offset + 4 * (l16 & 3);
        const int j = q8_offset >> 1;
        const int q8_word = l16 & 3;
        for (int bi = bi0 + (lane >> 4); bi < bi1; bi += 2) {
            const uint8_t *base = col + (size_t)bi * 144;
            const float d = or_f16_to_f32(rd16(base));
            const float minv = or_f16_to_f32(rd16(base + 2));
            const uint8_t *sc = base + 4;
            const uint8_t *qs = base + 16;
            const int32_t v0 = rd32(qs + q4_offset);
            const int32_t v1 = rd32(qs + q4_offset + 16);
            uint16_t sc16[6];
            for (int i = 0; i < 6; i++) sc16[i] = rd16(sc + 2 * i);
            uint16_t aux0, aux1;
            if (j < 2) {
                aux0 = sc16[j] & 0x3f3f;
                aux1 = sc16[j + 2] & 0x3f3f;
            } else {
                aux0 = (uint16_t)(((sc16[j + 2] >> 0) & 0x0f0f) | ((sc16[j - 2] & 0xc0c0) >> 2));
                aux1 = (uint16_t)(((sc16[j + 2] >> 4) & 0x0f0f) | ((sc16[j] & 0xc0c0) >> 2));
            }
            const int sc0 = aux0 & 0xff, sc1 = aux0 >> 8;
            const int m0 = aux1 & 0xff, m1 = aux1 >> 8;
            const int lb = bi - bi0;
            const int8_t *qb0 = q8 + (lb * 8 + q8_offset) * 32;
            const int8_t *qb1 = qb0 + 32;
            const int32_t ua0 = rd32(qb0 + 4 * q8_word), ua1 = rd32(qb0 + 4 * q8_word + 16);
            const int32_t ub0 = rd32(qb1 + 4 * q8_word), ub1 = rd32(qb1 + 4 * q8_word + 16);
            const int32_t dot0 = dp4a(v0 & 0x0f0f0f0f, ua0, dp4a(v1 & 0x0f0f0f0f, ua1, 0));
            const int32_t dot1 = dp4a((v0 >> 4) & 0x0f0f0f0f, ub0,
                                      dp4a((v1 >> 4) & 0x0f0f0f0f, ub1, 0));
            const int32_t sum0 = dp4a(0x01010101, ua0, dp4a(0x01010101, ua1, 0));
            const int32_t sum1 = dp4a(0x01010101, ub0, dp4a(0x01010101, ub1, 0));
            const float d8a = d8[lb * 8 + q8_offset];
            const float d8b = d8[lb * 8 + q8_offset + 1];
            a += d * (d8a * (float)(dot0 * sc0) + d8b * (float)(dot1 * sc1));
            a -= minv * (d8a * (float)(sum0 * m0) + d8b * (float)(sum1 * m1));
        }
        acc[lane] = a;
    }
    return warp_sum32(acc);
}

/* kernels/gemv.cu:367-373 gemv_apply_res, then the bias add of the callers */
static float epilogue(float acc, int j, float *out, int use_bias,
                      const float *bias, int use_res, const float *residual) {
    if (use_res == 1) acc += residual[j];
    else if (use_res == 2) acc += out[j];
    if (use_bias) acc += bias[j];
    return acc;
}

void or_gemv_q4k_q8(const uint8_t *w, const int8_t *xq, const float *xd,
                    float *out, int n_rows, int n_cols, int col_bytes,
                    int use_bias, const float *bias, int use_res,
                    const float *residual) {
    const int nsb = n_rows / 256; /* floor: the reference ignores a tail */
    for (int j = 0; j < n_cols; j++) {
        const float acc = dot_q4k_warp(w + (size_t)j * col_bytes, xq, xd, 0, nsb);
        out[j] = epilogue(acc, j, out, use_bias, bias, use_res, residual);
    }
}

void or_gemv_q4k_q8_splitk(const uint8_t *w, const int8_t *xq,
                           const float *xd, float *partial, int n_rows,
                           int n_cols, int col_bytes, int n_split) {
    const int nb = n_rows / 256;
    for (int s = 0; s < n_split; s++) {
        const int sb0 = (nb * s) / n_split, sb1 = (nb * (s + 1)) / n_split;
        const int mid = (sb0 + sb1 + 1) / 2;
        for (int j = 0; j < n_cols; j++) {
            const uint8_t *col = w + (size_t)j * col_bytes;
            const float a0 = dot_q4k_warp(col, xq + sb0 * 256, xd + sb0 * 8, sb0, mid);
            const float a1 = dot_q4k_warp(col, xq + mid * 256, xd + mid * 8, mid, sb1);
            partial[(size_t)s * n_cols + j] = a0 + a1;
        }
    }
}

void or_gemv_splitk_reduce(const float *partial, float *out, int n_cols,
                           int n_split, int use_bias, const float *bias,
                           int use_res, const float *residual) {
    for (int j = 0; j < n_cols; j++) {
        float acc = 0.f;
        for (int s = 0; s < n_split; s++) acc += partial[(size_t)s * n_cols + j];
        out[j] = epilogue(acc, j, out, use_bias, bias, use_res, residual);
    }
}

/* Two warps halve the super-blocks: [0, ceil(nb/2)) and [ceil(nb/2), nb). */
static float dot_q4k_halves(const uint8_t *col, const int8_t *xq,
                            const float *xd, int nb) {
    const int split = (nb + 1) / 2;
    const float a0 = dot_q4k_warp(col, xq, xd, 0, split);
    const float a1 = dot_q4k_warp(col, xq + split * 256, xd + split * 8, split, nb);
    return a0 + a1;
}

void or_gemv_q4k_pair(const uint8_t *wa, const uint8_t *wb, const int8_t *xq,
                      const float *xd, float *out_a, float *out_b, int n_rows,
                      int n_a, int n_b, int col_bytes, int use_bias,
                      const float *ba, const float *bb) {
    const int nb = n_rows / 256;
    for (int j = 0; j < n_a + n_b; j++) {
        const int is_a = j < n_a;
        const int oj = is_a ? j : j - n_a;
        const uint8_t *col = (is_a ? wa : wb) + (size_t)oj * col_bytes;
        float acc = dot_q4k_halves(col, xq, xd, nb);
        if (use_bias) acc += (is_a ? ba : bb)[oj];
        (is_a ? out_a : out_b)[oj] = acc;
    }
}

void or_gemv_q4k_dual(const uint8_t *wa, const uint8_t *wb, const int8_t *xq,
                      const float *xd, float *out_a, float *out_b, int n_rows,
                      int n_cols, int col_bytes) {
    const int nb = n_rows / 256;
    for (int j = 0; j < n_cols; j++) {
        out_a[j] = dot_q4k_halves(wa + (size_t)j * col_bytes, xq, xd, nb);
        out_b[j] = dot_q4k_halves(wb + (size_t)j * col_bytes, xq, xd, nb);
    }
}

/* One column of a `ways`-warp cooperative Q4_K dot (gemv.cu:2440-2659). */
static float dot_q4k_ways(const uint8_t *col, const int8_t *xq,
                          const float *xd, int nb, int ways) {
    if (ways == 1) return dot_q4k_warp(col, xq, xd, 0, nb);
    if (ways == 2) return dot_q4k_halves(col, xq, xd, nb);
    float total = 0.f;
    for (int w = 0; w < ways; w++) {
        const int b0 = (nb * w) / ways, b1 = (nb * (w + 1)) / ways;
        float p = 0.f;
        if (b0 < b1) p = dot_q4k_warp(col, xq + b0 * 256, xd + b0 * 8, b0, b1);
        total += p;
    }
    return total;
}

static void ffn_cols(const uint8_t *gate, const uint8_t *up, const int8_t *xq,
                     const float *xd, float *out, int n_rows, int j0, int j1,
                     int col_bytes, int ways) {
    const int nb = n_rows / 256;
    for (int j = j0; j < j1; j++) {
        const float g = dot_q4k_ways(gate + (size_t)j * col_bytes, xq, xd, nb, ways);
        const float u = dot_q4k_ways(up + (size_t)j * col_bytes, xq, xd, nb, ways);
        out[j] = (g / (1.f + expf(-g))) * u;
    }
}

void or_gemv_q4k_ffn(const uint8_t *gate, const uint8_t *up, const int8_t *xq,
                     const float *xd, float *out, int n_rows, int n_cols,
                     int col_bytes, int ways) {
    ffn_cols(gate, up, xq, xd, out, n_rows, 0, n_cols, col_bytes, ways);
}

void or_gemv_q4k_qkv(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv,
                     const int8_t *xq, const float *xd, float *q, float *k,
                     float *v, int n_rows, int n_q, int n_k, int n_v,
                     int col_bytes, int use_bias, const float *bq,
                     const float *bk, const float *bv) {
    const int nb = n_rows / 256;
    for (int j = 0; j < n_q + n_k + n_v; j++) {
        const uint8_t *w;
        float *out;
        const float *b;
        int oj;
        if (j < n_q) {
            w = wq; out = q; b = bq; oj = j;
        } else if (j < n_q + n_k) {
            w = wk; out = k; b = bk; oj = j - n_q;
        } else {
            w = wv; out = v; b = bv; oj = j - n_q - n_k;
        }
        float acc = dot_q4k_warp(w + (size_t)oj * col_bytes, xq, xd, 0, nb);
        if (use_bias) acc += b[oj];
        out[oj] = acc;
    }
}

/* ------------------------------------------------------------ Q6_K x Q8 */

/* kernels/gemv.cu:302-337 dot_q6_k_compact_q8_range over 212-byte blocks;
 * xq/xd point at super-block bi0. */
static float dot_q6c_warp(const uint8_t *col, const int8_t *xq, const float *xd,
                          int bi0, int bi1) {
    float acc[32];
    for (int lane = 0; lane < 32; lane++) {
        float a = 0.f;
        const int lane16 = lane & 15;
        for (int bi = bi0; bi < bi1; bi++) {
            const uint8_t *base = col + (size_t)bi * 212;
            const int8_t *sc = (const int8_t *)(base + 192);
            const float d = or_f16_to_f32(rd16(base + 208));
            const int local = (bi - bi0) * 256;
            const uint32_t ql = rdu32(base + 4 * lane);
            const int qh_word = 8 * (lane >> 4) + (lane & 7);
            uint32_t qh = rdu32(base + 128 + 4 * qh_word);
            qh >>= 2 * (lane16 >> 3);
            const int scale_offset = 8 * (lane >> 4) + (lane16 >> 2);
            const int q8_base = 4 * (lane >> 4) + (lane16 >> 3);
            for (int r = 0; r < 2; r++) {
                const uint32_t lo = (ql >> (4 * r)) & 0x0f0f0f0fu;
                const uint32_t hi = ((qh >> (4 * r)) << 4) & 0x30303030u;
                const int32_t wpack = vsubss4((int32_t)(lo | hi), 0x20202020);
                const int q8_block = q8_base + 2 * r;
                const int32_t apack = rd32(xq + local + 32 * q8_block + 4 * (lane & 7));
                const int32_t dot = dp4a(wpack, apack, 0);
                a += d * (float)sc[scale_offset + 4 * r] * xd[(local >> 5) + q8_block] *
                     (float)dot;
            }
        }
        acc[lane] = a;
    }
    return warp_sum32(acc);
}

void or_gemv_q6k_compact_q8(const uint8_t *w, const int8_t *xq,
                            const float *xd, float *out, int n_rows,
                            int n_cols, int col_bytes, int use_bias,
                            const float *bias, int use_res,
                            const float *residual) {
    const int nsb = n_rows / 256;
    for (int j = 0; j < n_cols; j++) {
        const float acc = dot_q6c_warp(w + (size_t)j * col_bytes, xq, xd, 0, nsb);
        out[j] = epilogue(acc, j, out, use_bias, bias, use_res, residual);
    }
}

static void q6_kway_cols(const uint8_t *w, const int8_t *xq, const float *xd,
                         float *out, int n_rows, int j0, int j1, int col_bytes,
                         int ways, int use_bias, const float *bias, int use_res,
                         const float *residual) {
    const int nsb = n_rows / 256;
    for (int j = j0; j < j1; j++) {
        const uint8_t *col = w + (size_t)j * col_bytes;
        float total = 0.f;
        for (int wp = 0; wp < ways; wp++) {
            const int b0 = (nsb * wp) / ways, b1 = (nsb * (wp + 1)) / ways;
            float p = 0.f;
            if (b0 < b1) p = dot_q6c_warp(col, xq + b0 * 256, xd + b0 * 8, b0, b1);
            total += p;
        }
        out[j] = epilogue(total, j, out, use_bias, bias, use_res, residual);
    }
}

void or_gemv_q6k_compact_q8_kway(const uint8_t *w, const int8_t *xq,
                                 const float *xd, float *out, int n_rows,
                                 int n_cols, int col_bytes, int ways,
                                 int use_bias, const float *bias, int use_res,
                                 const float *residual) {
    q6_kway_cols(w, xq, xd, out, n_rows, 0, n_cols, col_bytes, ways, use_bias,
                 bias, use_res, residual);
}

void or_gemv_q6k_compact_q8_splitk(const uint8_t *w, const int8_t *xq,
                                   const float *xd, float *partial,
                                   int n_rows, int n_cols, int col_bytes,
                                   int n_split) {
    const int nsb = n_rows / 256;
    for (int s = 0; s < n_split; s++) {
        const int b0 = (nsb * s) / n_split, b1 = (nsb * (s + 1)) / n_split;
        for (int j = 0; j < n_cols; j++)
            partial[(size_t)s * n_cols + j] =
                dot_q6c_warp(w + (size_t)j * col_bytes, xq + b0 * 256, xd + b0 * 8, b0, b1);
    }
}

/* kernels/gemv.cu:233-264 dot_q6_k_col_xs_range + :405-438 gemv_q6_k */
void or_gemv_q6k_f32(const uint8_t *w, const float *x, float *out, int n_rows,
                     int n_cols, int col_bytes, int use_bias,
                     const float *bias, int use_res, const float *residual) {
    const int nsb = n_rows / 256;
    for (int j = 0; j < n_cols; j++) {
        const uint8_t *col = w + (size_t)j * col_bytes;
        float acc[32];
        for (int lane = 0; lane < 32; lane++) {
            float a = 0.f;
            for (int bi = 0; bi < nsb; bi++) {
                const uint8_t *base = col + (size_t)bi * 210;
                const uint8_t *ql = base, *qh = base + 128;
                const int8_t *sc = (const int8_t *)(base + 192);
                const float d = or_f16_to_f32(rd16(base + 208));
                const float *xb = x + bi * 256;
                for (int n = 0; n < 2; n++) {
                    const int ql_i = n * 64, qh_i = n * 32, sc_i = n * 8, y0 = n * 128;
                    const int is = lane / 16;
                    const int q1 = (int)((ql[ql_i + lane] & 0xF) | (((qh[qh_i + lane] >> 0) & 3) << 4)) - 32;
                    const int q2 = (int)((ql[ql_i + 32 + lane] & 0xF) | (((qh[qh_i + lane] >> 2) & 3) << 4)) - 32;
                    const int q3 = (int)((ql[ql_i + lane] >> 4) | (((qh[qh_i + lane] >> 4) & 3) << 4)) - 32;
                    const int q4 = (int)((ql[ql_i + 32 + lane] >> 4) | (((qh[qh_i + lane] >> 6) & 3) << 4)) - 32;
                    a += d * (float)sc[sc_i + is] * (float)q1 * xb[y0 + lane];
                    a += d * (float)sc[sc_i + is + 2] * (float)q2 * xb[y0 + 32 + lane];
                    a += d * (float)sc[sc_i + is + 4] * (float)q3 * xb[y0 + 64 + lane];
                    a += d * (float)sc[sc_i + is + 6] * (float)q4 * xb[y0 + 96 + lane];
                }
            }
            acc[lane] = a;
        }
        out[j] = epilogue(warp_sum32(acc), j, out, use_bias, bias, use_res, residual);
    }
}

void or_q6k_compact_repack(const uint8_t *raw, uint8_t *out, int n_rows,
                           int n_cols, int col_bytes) {
    const int nb = n_rows / 256;
    const size_t ccb = (size_t)nb * 212;
    memset(out, 0, (size_t)n_cols * ccb);
    for (int c = 0; c < n_cols; c++)
        for (int bi = 0; bi < nb; bi++)
            memcpy(out + c * ccb + (size_t)bi * 212, raw + (size_t)c * col_bytes + (size_t)bi * 210, 210);
}

/* --------------------------------------------------------------- fp64 truth */

void or_gemv_q4k_q8_f64(const uint8_t *w, const int8_t *xq, const float *xd,
                        double *out, double *rowabs, int n_rows, int n_cols,
                        int col_bytes) {
    const int nsb = n_rows / 256;
    int32_t *dots = malloc(sizeof(int32_t) * 8 * (nsb > 0 ? nsb : 1));
    int32_t *sums = malloc(sizeof(int32_t) * 8 * (nsb > 0 ? nsb : 1));
    for (int j = 0; j < n_cols; j++) {
        const uint8_t *col = w + (size_t)j * col_bytes;
        or_q4k_block_dots(col, xq, nsb, dots, sums);
        double y = 0.0, a = 0.0;
        for (int bi = 0; bi < nsb; bi++) {
            const uint8_t *base = col + (size_t)bi * 144;
            const double d = or_f16_to_f32(rd16(base));
            const double dmin = or_f16_to_f32(rd16(base + 2));
            for (int g = 0; g < 8; g++) {
                int sc, m;
                scale_min_k4(g, base + 4, &sc, &m);
                const double t1 = d * sc * (double)xd[bi * 8 + g] * dots[bi * 8 + g];
                const double t2 = dmin * m * (double)xd[bi * 8 + g] * sums[bi * 8 + g];
                y += t1 - t2;
                a += fabs(t1) + fabs(t2);
            }
        }
        out[j] = y;
        if (rowabs) rowabs[j] = a;
    }
    free(dots);
    free(sums);
}

void or_gemv_q6k_q8_f64(const uint8_t *w, int block_bytes, const int8_t *xq,
                        const float *xd, double *out, double *rowabs,
                        int n_rows, int n_cols, int col_bytes) {
    const int nsb = n_rows / 256;
    int32_t *dots = malloc(sizeof(int32_t) * 16 * (nsb > 0 ? nsb : 1));
    for (int j = 0; j < n_cols; j++) {
        const uint8_t *col = w + (size_t)j * col_bytes;
        or_q6k_block_dots(col, block_bytes, xq, nsb, dots);
        double y = 0.0, a = 0.0;
        for (int bi = 0; bi < nsb; bi++) {
            const uint8_t *base = col + (size_t)bi * block_bytes;
            const double d = or_f16_to_f32(rd16(base + 208));
            for (int g = 0; g < 16; g++) {
                const double t = d * (int8_t)base[192 + g] * (double)xd[bi * 8 + g / 2] *
                                 dots[bi * 16 + g];
                y += t;
                a += fabs(t);
            }
        }
        out[j] = y;
        if (rowabs) rowabs[j] = a;
    }
    free(dots);
}

void or_gemv_q6k_f32_f64(const uint8_t *w, const float *x, double *out,
                         double *rowabs, int n_rows, int n_cols,
                         int col_bytes) {
    const int nsb = n_rows / 256;
    for (int j = 0; j < n_cols; j++) {
        const uint8_t *col = w + (size_t)j * col_bytes;
        double y = 0.0, a = 0.0;
        for (int bi = 0; bi < nsb; bi++) {
            const uint8_t *base = col + (size_t)bi * 210;
            const double d = or_f16_to_f32(rd16(base + 208));
            for (int v = 0; v < 256; v++) {
                const double t = d * (int8_t)base[192 + v / 16] * q6_value(base, v) *
                                 (double)x[bi * 256 + v];
                y += t;
                a += fabs(t);
            }
        }
        out[j] = y;
        if (rowabs) rowabs[j] = a;
    }
}

/* ------------------------------------------------------- Q8_0 / Q5_0 */

static int q5_0_value(const uint8_t *blk, int v) {
    const uint32_t qh = rdu32(blk + 2);
    const uint8_t *qs = blk + 6;
    const int t = v & 15;
    int q;
    if (v < 16) q = (qs[t] & 0x0F) | (int)(((qh >> t) << 4) & 0x10u);
    else q = (qs[t] >> 4) | (int)((qh >> (t + 12)) & 0x10u);
    return q - 16;
}

/* dot_q8_0_col_q8_range for one lane's blocks [bi0 + lane : bi1 : 32] */
static float q8_0_lane(const uint8_t *col, const int8_t *xq, const float *xd,
                       int bi0, int bi1, int lane) {
    float acc = 0.f;
    for (int bi = bi0 + lane; bi < bi1; bi += 32) {
        const uint8_t *base = col + (size_t)bi * 34;
        const float dw = or_f16_to_f32(rd16(base));
        int32_t sum = 0;
        for (int t = 0; t < 32; t += 4)
            sum = dp4a(rd32(base + 2 + t), rd32(xq + bi * 32 + t), sum);
        acc += dw * xd[bi] * (float)sum;
    }
    return acc;
}

void or_gemv_q8_0_q8(const uint8_t *w, const int8_t *xq, const float *xd,
                     float *out, int n_rows, int n_cols, int col_bytes,
                     int use_bias, const float *bias, int use_res,
                     const float *residual) {
    const int nb = n_rows / 32;
    for (int j = 0; j < n_cols; j++) {
        const uint8_t *col = w + (size_t)j * col_bytes;
        float acc[32];
        for (int lane = 0; lane < 32; lane++) acc[lane] = q8_0_lane(col, xq, xd, 0, nb, lane);
        out[j] = epilogue(warp_sum32(acc), j, out, use_bias, bias, use_res, residual);
    }
}

void or_gemv_q8_0_q8_splitk(const uint8_t *w, const int8_t *xq,
                            const float *xd, float *partial, int n_rows,
                            int n_cols, int col_bytes, int n_split) {
    const int nb = n_rows / 32;
    for (int s = 0; s < n_split; s++) {
        const int bi0 = nb * s / n_split, bi1 = nb * (s + 1) / n_split;
        for (int j = 0; j < n_cols; j++) {
            float acc[32];
            for (int lane = 0; lane < 32; lane++)
                acc[lane] = q8_0_lane(w + (size_t)j * col_bytes, xq, xd, bi0, bi1, lane);
            partial[(size_t)s * n_cols + j] = bi0 >= bi1 ? 0.f : warp_sum32(acc);
        }
    }
}

void or_gemv_q8_0_f32_splitk(const uint8_t *w, const float *x, float *partial,
                             int n_rows, int n_cols, int col_bytes,
                             int n_split) {
    const int nb = n_rows / 32;
    for (int s = 0; s < n_split; s++) {
        const int bi0 = nb * s / n_split, bi1 = nb * (s + 1) / n_split;
        for (int j = 0; j < n_cols; j++) {
            const uint8_t *col = w + (size_t)j * col_bytes;
            float acc[32];
            for (int lane = 0; lane < 32; lane++) {
                float a = 0.f;
                for (int bi = bi0 + lane; bi < bi1; bi += 32) {
                    const uint8_t *base = col + (size_t)bi * 34;
                    const float d = or_f16_to_f32(rd16(base));
                    const int8_t *qs = (const int8_t *)(base + 2);
                    for (int t = 0; t < 32; t++) a += (float)qs[t] * d * x[bi * 32 + t];
                }
                acc[lane] = a;
            }
            partial[(size_t)s * n_cols + j] = bi0 >= bi1 ? 0.f : warp_sum32(acc);
        }
    }
}

/* one lane of gemv_q5_0 / gemv_q5_0_splitk over blocks [bi0 + lane : bi1 : 32] */
static float q5_0_lane(const uint8_t *col, const float *x, int bi0, int bi1, int lane) {
    float acc = 0.f;
    for (int bi = bi0 + lane; bi < bi1; bi += 32) {
        const uint8_t *base = col + (size_t)bi * 22;
        const float d = or_f16_to_f32(rd16(base));
        const uint32_t qh = rdu32(base + 2);
        const uint8_t *qs = base + 6;
        const float *xs = x + bi * 32;
        for (int t = 0; t < 16; t++) {
            const int x0 = (qs[t] & 0x0F) | (int)(((qh >> t) << 4) & 0x10u);
            const int x1 = (qs[t] >> 4) | (int)((qh >> (t + 12)) & 0x10u);
            acc += (float)(x0 - 16) * d * xs[t];
            acc += (float)(x1 - 16) * d * xs[16 + t];
        }
    }
    return acc;
}

void or_gemv_q5_0_f32(const uint8_t *w, const float *x, float *out,
                      int n_rows, int n_cols, int col_bytes, int use_bias,
                      const float *bias, int use_res, const float *residual) {
    const int nb = n_rows / 32;
    for (int j = 0; j < n_cols; j++) {
        float acc[32];
        for (int lane = 0; lane < 32; lane++)
            acc[lane] = q5_0_lane(w + (size_t)j * col_bytes, x, 0, nb, lane);
        out[j] = epilogue(warp_sum32(acc), j, out, use_bias, bias, use_res, residual);
    }
}

void or_gemv_q5_0_f32_splitk(const uint8_t *w, const float *x, float *partial,
                             int n_rows, int n_cols, int col_bytes,
                             int n_split) {
    const int nb = n_rows / 32;
    for (int s = 0; s < n_split; s++) {
        const int bi0 = nb * s / n_split, bi1 = nb * (s + 1) / n_split;
        for (int j = 0; j < n_cols; j++) {
            float acc[32];
            for (int lane = 0; lane < 32; lane++)
                acc[lane] = q5_0_lane(w + (size_t)j * col_bytes, x, bi0, bi1, lane);
            partial[(size_t)s * n_cols + j] = bi0 >= bi1 ? 0.f : warp_sum32(acc);
        }
    }
}

void or_q8_0_block_sums(const uint8_t *w, const int8_t *xq, int32_t *sums,
                        int n_rows, int n_cols, int col_bytes) {
    const int nb = n_rows / 32;
    for (int j = 0; j < n_cols; j++)
        for (int bi = 0; bi < nb; bi++) {
            const int8_t *qs = (const int8_t *)(w + (size_t)j * col_bytes + (size_t)bi * 34 + 2);
            int32_t s = 0;
            for (int t = 0; t < 32; t++) s += (int32_t)qs[t] * xq[bi * 32 + t];
            sums[(size_t)j * nb + bi] = s;
        }
}

void or_gemv_q8_0_q8_f64(const uint8_t *w, const int8_t *xq, const float *xd,
                         double *out, double *rowabs, int n_rows, int n_cols,
                         int col_bytes) {
    const int nb = n_rows / 32;
    for (int j = 0; j < n_cols; j++) {
        double y = 0.0, a = 0.0;
        for (int bi = 0; bi < nb; bi++) {
            const uint8_t *base = w + (size_t)j * col_bytes + (size_t)bi * 34;
            const double dw = or_f16_to_f32(rd16(base));
            const int8_t *qs = (const int8_t *)(base + 2);
            for (int t = 0; t < 32; t++) {
                const double v = dw * (double)xd[bi] * qs[t] * xq[bi * 32 + t];
                y += v;
                a += fabs(v);
            }
        }
        out[j] = y;
        if (rowabs) rowabs[j] = a;
    }
}

void or_gemv_q8_0_f32_f64(const uint8_t *w, const float *x, double *out,
                          double *rowabs, int n_rows, int n_cols,
                          int col_bytes) {
    const int nb = n_rows / 32;
    for (int j = 0; j < n_cols; j++) {
        double y = 0.0, a = 0.0;
        for (int bi = 0; bi < nb; bi++) {
            const uint8_t *base = w + (size_t)j * col_bytes + (size_t)bi * 34;
            const double d = or_f16_to_f32(rd16(base));
            for (int t = 0; t < 32; t++) {
                const double v = d * (int8_t)base[2 + t] * (double)x[bi * 32 + t];
                y += v;
                a += fabs(v);
            }
        }
        out[j] = y;
        if (rowabs) rowabs[j] = a;
    }
}

void or_gemv_q5_0_f32_f64(const uint8_t *w, const float *x, double *out,
                          double *rowabs, int n_rows, int n_cols,
                          int col_bytes) {
    const int nb = n_rows / 32;
    for (int j = 0; j < n_cols; j++) {
        double y = 0.0, a = 0.0;
        for (int bi = 0; bi < nb; bi++) {
            const uint8_t *base = w + (size_t)j * col_bytes + (size_t)bi * 22;
            const double d = or_f16_to_f32(rd16(base));
            for (int v = 0; v < 32; v++) {
                const double t = d * q5_0_value(base, v) * (double)x[bi * 32 + v];
                y += t;
                a += fabs(t);
            }
        }
        out[j] = y;
        if (rowabs) rowabs[j] = a;
    }
}

/* -------------------------------------------------------------- prefill GEMM */

/* common.cu:64-84: the 256 f32 weights of one Q4_K super-block */
static void dequant_q4k_f32(const uint8_t *base, float *dq) {
    const float d = or_f16_to_f32(rd16(base));
    const float minv = or_f16_to_f32(rd16(base + 2));
    const uint8_t *q = base + 16;
    for (int t = 0; t < 4; t++) {
        int sc, m;
        scale_min_k4(2 * t, base + 4, &sc, &m);
        const float d1 = d * (float)sc, m1 = minv * (float)m;
        scale_min_k4(2 * t + 1, base + 4, &sc, &m);
        const float d2 = d * (float)sc, m2 = minv * (float)m;
        for (int l = 0; l < 32; l++) {
            dq[t * 64 + l] = d1 * (float)(q[t * 32 + l] & 0xF) - m1;
            dq[t * 64 + 32 + l] = d2 * (float)(q[t * 32 + l] >> 4) - m2;
        }
    }
}

/* common.cu:164-186: the 256 f32 weights of one raw Q6_K super-block */
static void dequant_q6k_f32(const uint8_t *base, float *dq) {
    const uint8_t *ql = base, *qh = base + 128;
    const int8_t *sc = (const int8_t *)(base + 192);
    const float d = or_f16_to_f32(rd16(base + 208));
    for (int n = 0; n < 2; n++) {
        const int ql_i = n * 64, qh_i = n * 32, sc_i = n * 8, y0 = n * 128;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((ql[ql_i + l] & 0xF) | (((qh[qh_i + l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((ql[ql_i + 32 + l] & 0xF) | (((qh[qh_i + l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[ql_i + l] >> 4) | (((qh[qh_i + l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[ql_i + 32 + l] >> 4) | (((qh[qh_i + l] >> 6) & 3) << 4)) - 32;
            dq[y0 + l] = d * (float)sc[sc_i + is] * (float)q1;
            dq[y0 + 32 + l] = d * (float)sc[sc_i + is + 2] * (float)q2;
            dq[y0 + 64 + l] = d * (float)sc[sc_i + is + 4] * (float)q3;
            dq[y0 + 96 + l] = d * (float)sc[sc_i + is + 6] * (float)q4;
        }
    }
}

static void gemm_ref_order(const uint8_t *w, const float *x, float *out, int n_rows,
                           int n_cols, int col_bytes, int n_tok, int block_bytes,
                           void (*deq)(const uint8_t *, float *)) {
    const int nb = n_rows / 256;
    float *dq = (float *)malloc((size_t)nb * 256 * sizeof(float));
    float acc[32];
    for (int j = 0; j < n_cols; j++) {
        const uint8_t *col = w + (size_t)j * col_bytes;
        for (int bi = 0; bi < nb; bi++) deq(col + (size_t)bi * block_bytes, dq + bi * 256);
        for (int t = 0; t < n_tok; t++) {
            const float *xt = x + (size_t)t * n_rows;
            for (int l = 0; l < 32; l++) {
                float a = 0.f;
                for (int bi = 0; bi < nb; bi++)
                    for (int i = l; i < 256; i += 32) a += dq[bi * 256 + i] * xt[bi * 256 + i];
                acc[l] = a;
            }
            out[(size_t)t * n_cols + j] = warp_sum32(acc);
        }
    }
    free(dq);
}

void or_gemm_q4k(const uint8_t *w, const float *x, float *out, int n_rows,
                 int n_cols, int col_bytes, int n_tok) {
    gemm_ref_order(w, x, out, n_rows, n_cols, col_bytes, n_tok, 144, dequant_q4k_f32);
}

void or_gemm_q6k(const uint8_t *w, const float *x, float *out, int n_rows,
                 int n_cols, int col_bytes, int n_tok) {
    gemm_ref_order(w, x, out, n_rows, n_cols, col_bytes, n_tok, 210, dequant_q6k_f32);
}

/* ops.cu:507-529 block_max / block_sum over 128 threads (halving tree) */
static float block_tree128(float *buf, int is_max) {
    for (int s = 64; s > 0; s >>= 1)
        for (int i = 0; i < s; i++)
            buf[i] = is_max ? fmaxf(buf[i], buf[i + s]) : buf[i] + buf[i + s];
    return buf[0];
}

void or_attn_prefill(const float *q, const uint16_t *k_cache,
                     const uint16_t *v_cache, float *out, int n_head, int n_kv,
                     int head_dim, int pos0, int n_q, float scale) {
    const int rep = n_head / n_kv, stride = n_kv * head_dim, NT = 128, TILE = 64;
    float scores[64], buf[128];
    for (int qi = 0; qi < n_q; qi++)
        for (int h = 0; h < n_head; h++) {
            const int kv_h = h / rep, seq_len = pos0 + qi + 1;
            const float *qh = q + (size_t)qi * n_head * head_dim + (size_t)h * head_dim;
            float m = -1e30f, l = 0.f, acc0[128], acc1[128];
            for (int t = 0; t < NT; t++) acc0[t] = acc1[t] = 0.f;
            for (int t0 = 0; t0 < seq_len; t0 += TILE) {
                const int tlen = seq_len - t0 < TILE ? seq_len - t0 : TILE;
                for (int t = 0; t < tlen; t++) {
                    const uint16_t *row = k_cache + (size_t)(t0 + t) * stride + (size_t)kv_h * head_dim;
                    float dot = 0.f;
                    for (int d = 0; d < head_dim; d++) dot += qh[d] * or_f16_to_f32(row[d]);
                    scores[t] = dot * scale;
                }
                for (int tid = 0; tid < NT; tid++) buf[tid] = tid < tlen ? scores[tid] : -1e30f;
                const float m_new = fmaxf(m, block_tree128(buf, 1));
                const float alpha = expf(m - m_new);
                for (int tid = 0; tid < NT; tid++) {
                    float e = 0.f;
                    if (tid < tlen) {
                        e = expf(scores[tid] - m_new);
                        scores[tid] = e;
                    }
                    buf[tid] = e;
                }
                const float tile_l = block_tree128(buf, 0);
                for (int tid = 0; tid < NT; tid++) {
                    const int d0 = tid, d1 = tid + NT;
                    acc0[tid] *= alpha;
                    if (d1 < head_dim) acc1[tid] *= alpha;
                    if (d0 < head_dim) {
                        float a0 = 0.f, a1 = 0.f;
                        for (int t = 0; t < tlen; t++) {
                            const uint16_t *vr = v_cache + (size_t)(t0 + t) * stride + (size_t)kv_h * head_dim;
                            a0 += scores[t] * or_f16_to_f32(vr[d0]);
                            if (d1 < head_dim) a1 += scores[t] * or_f16_to_f32(vr[d1]);
                        }
                        acc0[tid] += a0;
                        acc1[tid] += a1;
                    }
                }
                l = l * alpha + tile_l;
                m = m_new;
            }
            const float inv = 1.f / fmaxf(l, 1e-20f);
            float *oh = out + (size_t)qi * n_head * head_dim + (size_t)h * head_dim;
            for (int tid = 0; tid < NT; tid++) {
                if (tid < head_dim) oh[tid] = acc0[tid] * inv;
                if (tid + NT < head_dim) oh[tid + NT] = acc1[tid] * inv;
            }
        }
}

/* -------------------------------------------------------------- flash decode */

#define OR_ATTN_TILE 64
#define OR_FLASH_THREADS 128 /* cuda/decode.rs:109 block_threads */

/* kernels/ops.cu:548-571 kv_dot_q (head_dim % 4 == 0 branch) */
static float kv_dot_q(const float *qh, const uint16_t *row, int head_dim) {
    float dot = 0.f;
    if ((head_dim & 3) == 0) {
        for (int d = 0; d < head_dim; d += 4) {
            const float k0 = or_f16_to_f32(row[d]), k1 = or_f16_to_f32(row[d + 1]);
            const float k2 = or_f16_to_f32(row[d + 2]), k3 = or_f16_to_f32(row[d + 3]);
            dot += qh[d] * k0 + qh[d + 1] * k1 + qh[d + 2] * k2 + qh[d + 3] * k3;
        }
    } else {
        for (int d = 0; d < head_dim; d++) dot += qh[d] * or_f16_to_f32(row[d]);
    }
    return dot;
}

/* kernels/ops.cu:519-529 block_sum: shared-memory halving tree. */
static float block_sum128(float *buf) {
    for (int s = OR_FLASH_THREADS / 2; s > 0; s >>= 1)
        for (int t = 0; t < s; t++) buf[t] += buf[t + s];
    return buf[0];
}

static void flash_partial_heads(const float *q, const uint16_t *k_cache,
                                const uint16_t *v_cache, float *partial, int n_head,
                                int n_kv, int head_dim, int pos0, int n_split,
                                float scale, int h0, int h1);

void or_flash_partial(const float *q, const uint16_t *k_cache,
                      const uint16_t *v_cache, float *partial, int n_head,
                      int n_kv, int head_dim, int pos0, int n_split,
                      float scale) {
    flash_partial_heads(q, k_cache, v_cache, partial, n_head, n_kv, head_dim, pos0,
                        n_split, scale, 0, n_head);
}

static void flash_partial_heads(const float *q, const uint16_t *k_cache,
                                const uint16_t *v_cache, float *partial, int n_head,
                                int n_kv, int head_dim, int pos0, int n_split,
                                float scale, int h0, int h1) {
    const int rep = n_head / n_kv;
    const int stride = n_kv * head_dim;
    const int seq_len = pos0 + 1;
    const int chunk = (seq_len + n_split - 1) / n_split;
    float scores[OR_ATTN_TILE];
    float buf[OR_FLASH_THREADS];
    float *acc = malloc(sizeof(float) * head_dim);
    for (int h = h0; h < h1; h++) {
        const int kv_h = h / rep;
        const float *qh = q + (size_t)h * head_dim;
        for (int s = 0; s < n_split; s++) {
            const int t_begin = s * chunk;
            int t_end = t_begin + chunk;
            if (t_end > seq_len) t_end = seq_len;
            float m = -1e30f, l = 0.f;
            for (int d = 0; d < head_dim; d++) acc[d] = 0.f;
            for (int t0 = t_begin; t0 < t_end; t0 += OR_ATTN_TILE) {
                int tlen = t_end - t0;
                if (tlen > OR_ATTN_TILE) tlen = OR_ATTN_TILE;
                float tile_m = -1e30f;
                for (int t = 0; t < tlen; t++) {
                    const uint16_t *row = k_cache + (size_t)(t0 + t) * stride + (size_t)kv_h * head_dim;
                    scores[t] = kv_dot_q(qh, row, head_dim) * scale;
                    tile_m = fmaxf(tile_m, scores[t]);
                }
                const float m_new = fmaxf(m, tile_m);
                const float alpha = expf(m - m_new);
                for (int t = 0; t < OR_FLASH_THREADS; t++) buf[t] = 0.f;
                for (int t = 0; t < tlen; t++) {
                    const float e = expf(scores[t] - m_new);
                    scores[t] = e;
                    buf[t] = e; /* thread t holds score t (tile < threads) */
                }
                const float tile_l = block_sum128(buf);
                for (int d = 0; d < head_dim; d++) {
                    float a0 = 0.f;
                    for (int t = 0; t < tlen; t++) {
                        const uint16_t *vrow = v_cache + (size_t)(t0 + t) * stride + (size_t)kv_h * head_dim;
                        a0 += scores[t] * or_f16_to_f32(vrow[d]);
                    }
                    acc[d] *= alpha;
                    acc[d] += a0;
                }
                l = l * alpha + tile_l;
                m = m_new;
            }
            float *base = partial + ((size_t)h * n_split + s) * (size_t)(2 + head_dim);
            base[0] = m;
            base[1] = l;
            for (int d = 0; d < head_dim; d++) base[2 + d] = acc[d];
        }
    }
    free(acc);
}

void or_flash_reduce(const float *partial, float *out, int n_head,
                     int head_dim, int n_split) {
    const int po = 2 + head_dim;
    for (int h = 0; h < n_head; h++) {
        float m = -1e30f;
        for (int s = 0; s < n_split; s++)
            m = fmaxf(m, partial[((size_t)h * n_split + s) * po]);
        for (int d = 0; d < head_dim; d++) {
            float l = 0.f, acc = 0.f;
            for (int s = 0; s < n_split; s++) {
                const float *base = partial + ((size_t)h * n_split + s) * po;
                const float alpha = expf(base[0] - m);
                l += alpha * base[1];
                acc += alpha * base[2 + d];
            }
            out[(size_t)h * head_dim + d] = acc / fmaxf(l, 1e-20f);
        }
    }
}

void or_attn_f64(const float *q, const uint16_t *k_cache,
                 const uint16_t *v_cache, double *out, int n_head, int n_kv,
                 int head_dim, int seq_len, float scale) {
    const int rep = n_head / n_kv;
    const int stride = n_kv * head_dim;
    double *sc = malloc(sizeof(double) * (seq_len > 0 ? seq_len : 1));
    for (int h = 0; h < n_head; h++) {
        const int kv_h = h / rep;
        double mx = -INFINITY;
        for (int t = 0; t < seq_len; t++) {
            const uint16_t *row = k_cache + (size_t)t * stride + (size_t)kv_h * head_dim;
            double s = 0.0;
            for (int d = 0; d < head_dim; d++)
                s += (double)q[h * head_dim + d] * or_f16_to_f32(row[d]);
            sc[t] = s * (double)scale;
            if (sc[t] > mx) mx = sc[t];
        }
        double l = 0.0;
        for (int t = 0; t < seq_len; t++) {
            sc[t] = exp(sc[t] - mx);
            l += sc[t];
        }
        for (int d = 0; d < head_dim; d++) {
            double a = 0.0;
            for (int t = 0; t < seq_len; t++)
                a += sc[t] * or_f16_to_f32(v_cache[(size_t)t * stride + (size_t)kv_h * head_dim + d]);
            out[(size_t)h * head_dim + d] = a / l;
        }
    }
    free(sc);
}

/* ------------------------------------------------------- decode-step glue */

/* kernels/common.cu:64-84 dequant_q4_k_block_smem, one value:
 * (d*sc)*q - dmin*m; both products are exact in fp32. */
static float q4k_dequant_value(const uint8_t *blk, int v) {
    const float d = or_f16_to_f32(rd16(blk)), dmin = or_f16_to_f32(rd16(blk + 2));
    int sc, m;
    scale_min_k4(v >> 5, blk + 4, &sc, &m);
    const int t = v >> 6, l = v & 31;
    const uint8_t qb = blk[16 + 32 * t + l];
    const int q = ((v >> 5) & 1) ? (qb >> 4) : (qb & 0xF);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    return d1 * (float)q - m1;
}

void or_embed_row(const uint8_t *table, int block_bytes, int token, int n_rows,
                  int col_bytes, float *out) {
    const uint8_t *col = table + (size_t)token * col_bytes;
    const int nb = n_rows / 256;
    for (int bi = 0; bi < nb; bi++) {
        const uint8_t *blk = col + (size_t)bi * block_bytes;
        for (int v = 0; v < 256; v++) {
            if (block_bytes == 144) {
                out[bi * 256 + v] = q4k_dequant_value(blk, v);
            } else { /* kernels/common.cu:164-186: (d*sc)*q */
                const float d = or_f16_to_f32(rd16(blk + 208));
                out[bi * 256 + v] = d * (float)(int8_t)blk[192 + v / 16] * (float)q6_value(blk, v);
            }
        }
    }
}

void or_rms_norm(const float *x, const float *w, float *out, int n, float eps) {
    float buf[256];
    for (int t = 0; t < 256; t++) {
        float local = 0.f;
        /* the reference is compiled with fmad=true (cuda/device.rs:114): the
           square-accumulate is one fused multiply-add */
        for (int i = t; i < n; i += 256) local = fmaf(x[i], x[i], local);
        buf[t] = local;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int t = 0; t < s; t++) buf[t] += buf[t + s];
    const float scale = 1.0f / sqrtf(buf[0] / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

void or_rope_neox(float *x, int n_heads, int head_dim, int pos, float theta) {
    const int half = head_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        float *base = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            const float freq = powf(theta, -2.f * (float)i / (float)head_dim);
            const float ang = (float)pos * freq;
            const float c = cosf(ang), s = sinf(ang);
            const float x0 = base[i], x1 = base[i + half];
            base[i] = x0 * c - x1 * s;
            base[i + half] = x0 * s + x1 * c;
        }
    }
}

void or_f32_to_f16_array(const float *src, uint16_t *dst, int n) {
    for (int i = 0; i < n; i++) dst[i] = or_f32_to_f16_halfup(src[i]);
}

/* kernels/ops.cu:573-599 argmax_f32 as layer.rs:2248-2255 launches it: one
 * block of 256 threads.  Thread t scans i = t, t+256, ... keeping the first
 * strict maximum above -1e30 (index 0 if none); the slots then merge in the
 * halving tree where slot t takes slot t+s only if strictly greater. */
int or_argmax(const float *x, int n) {
    enum { T = 256 };
    float bv[T];
    int bi[T];
    for (int t = 0; t < T; t++) {
        float best_v = -1e30f;
        int best_i = 0;
        for (int i = t; i < n; i += T) {
            const float v = x[i];
            if (v > best_v) { best_v = v; best_i = i; }
        }
        bv[t] = best_v;
        bi[t] = best_i;
    }
    for (int s = T / 2; s > 0; s >>= 1)
        for (int t = 0; t < s; t++)
            if (bv[t + s] > bv[t]) { bv[t] = bv[t + s]; bi[t] = bi[t + s]; }
    return bi[0];
}

/* ------------------------------------------------------ CPU baseline (MT) */

typedef struct {
    int kind; /* 0 q4k, 1 ffn, 2 q6 kway, 3 flash partial over heads */
    const uint8_t *w, *w2;
    const int8_t *xq;
    const float *xd;
    float *out;
    int n_rows, j0, j1, col_bytes, ways;
    /* flash: q = (const float *)w, K/V = kc/vc, partial = out */
    const uint16_t *kc, *vc;
    int n_head, n_kv, head_dim, pos0, n_split;
    float scale;
} or_job;

static void *or_worker(void *arg) {
    or_job *jb = (or_job *)arg;
    const int nsb = jb->n_rows / 256;
    if (jb->kind == 0) {
        for (int j = jb->j0; j < jb->j1; j++)
            jb->out[j] = dot_q4k_warp(jb->w + (size_t)j * jb->col_bytes, jb->xq, jb->xd, 0, nsb);
    } else if (jb->kind == 1) {
        ffn_cols(jb->w, jb->w2, jb->xq, jb->xd, jb->out, jb->n_rows, jb->j0, jb->j1,
                 jb->col_bytes, jb->ways);
    } else if (jb->kind == 2) {
        q6_kway_cols(jb->w, jb->xq, jb->xd, jb->out, jb->n_rows, jb->j0, jb->j1,
                     jb->col_bytes, jb->ways, 0, NULL, 0, NULL);
    } else {
        flash_partial_heads((const float *)jb->w, jb->kc, jb->vc, jb->out, jb->n_head,
                            jb->n_kv, jb->head_dim, jb->pos0, jb->n_split, jb->scale,
                            jb->j0, jb->j1);
    }
    return NULL;
}

static void or_run_mt(or_job proto, int n_cols, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    or_job jobs[256];
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = proto;
        jobs[t].j0 = (int)((long long)n_cols * t / nthreads);
        jobs[t].j1 = (int)((long long)n_cols * (t + 1) / nthreads);
        if (nthreads == 1) or_worker(&jobs[t]);
        else pthread_create(&th[t], NULL, or_worker, &jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
}

void or_gemv_q4k_q8_mt(const uint8_t *w, const int8_t *xq, const float *xd,
                       float *out, int n_rows, int n_cols, int col_bytes,
                       int nthreads) {
    or_job p = {.kind = 0, .w = w, .xq = xq, .xd = xd, .out = out, .n_rows = n_rows,
                .col_bytes = col_bytes, .ways = 1};
    or_run_mt(p, n_cols, nthreads);
}

void or_gemv_q4k_ffn_mt(const uint8_t *gate, const uint8_t *up,
                        const int8_t *xq, const float *xd, float *out,
                        int n_rows, int n_cols, int col_bytes, int nthreads) {
    or_job p = {.kind = 1, .w = gate, .w2 = up, .xq = xq, .xd = xd, .out = out,
                .n_rows = n_rows, .col_bytes = col_bytes, .ways = 1};
    or_run_mt(p, n_cols, nthreads);
}

void or_gemv_q6k_compact_q8_kway_mt(const uint8_t *w, const int8_t *xq,
                                    const float *xd, float *out, int n_rows,
                                    int n_cols, int col_bytes, int ways,
                                    int nthreads) {
    or_job p = {.kind = 2, .w = w, .xq = xq, .xd = xd, .out = out, .n_rows = n_rows,
                .col_bytes = col_bytes, .ways = ways};
    or_run_mt(p, n_cols, nthreads);
}

/* or_flash_partial with the query heads partitioned over threads. */
void or_flash_partial_mt(const float *q, const uint16_t *k_cache,
                         const uint16_t *v_cache, float *partial, int n_head,
                         int n_kv, int head_dim, int pos0, int n_split,
                         float scale, int nthreads) {
    or_job p = {.kind = 3, .w = (const uint8_t *)q, .out = partial, .kc = k_cache,
                .vc = v_cache, .n_head = n_head, .n_kv = n_kv, .head_dim = head_dim,
                .pos0 = pos0, .n_split = n_split, .scale = scale};
    or_run_mt(p, n_head, nthreads > n_head ? n_head : nthreads);
}
