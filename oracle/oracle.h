/*
 * CPU oracle for the taraference batch-1 decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / CPU baseline.
 *
 * Every function restates the arithmetic of one reference kernel (cited as
 * path:line under crates/core/src/cuda/ of agkomyint/taraference v0.5.3) in
 * plain C.  The fp32 functions follow the reference's per-lane work split and
 * its warp_sum shuffle tree, so their summation order matches the reference
 * GPU kernels (up to the NVRTC fast-math contraction / __expf choices that a
 * CPU cannot reproduce).  The *_f64 functions are order-free fp64 "truth"
 * computed from the exact integer sums.
 *
 * Weight layout (reference naming): n_rows = K (input length), n_cols = N
 * (outputs).  Output column j occupies col_bytes bytes at w + j*col_bytes,
 * holding floor(n_rows/256) consecutive super-blocks.
 */
#ifndef TF_ORACLE_H
#define TF_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16_halfup(float f);

/* kernels/gemv.cu:43-65 quantize_q8_global */
void or_quantize_q8(const float *x, int8_t *q8, float *d8, int n_rows);

/* Exact integer stages.  For super-block bi and 32-value sub-block g:
 *   dots[(bi*8+g)] = sum q4 * q8,  sums[(bi*8+g)] = sum q8.        */
void or_q4k_block_dots(const uint8_t *col, const int8_t *q8, int nsb,
                       int32_t *dots, int32_t *sums);
/* Q6_K, per 16-value scale group g of super-block bi:
 *   dots[bi*16+g] = sum (q6-32) * q8                               */
void or_q6k_block_dots(const uint8_t *col, int block_bytes, const int8_t *q8,
                       int nsb, int32_t *dots);

/* kernels/gemv.cu:469-490 gemv_q4_k_global (one warp per column) */
void or_gemv_q4k_q8(const uint8_t *w, const int8_t *xq, const float *xd,
                    float *out, int n_rows, int n_cols, int col_bytes,
                    int use_bias, const float *bias, int use_res,
                    const float *residual);
/* kernels/gemv.cu:1877-1905 gemv_q4_k_global_splitk */
void or_gemv_q4k_q8_splitk(const uint8_t *w, const int8_t *xq,
                           const float *xd, float *partial, int n_rows,
                           int n_cols, int col_bytes, int n_split);
/* kernels/gemv.cu:2243-2263 gemv_splitk_reduce */
void or_gemv_splitk_reduce(const float *partial, float *out, int n_cols,
                           int n_split, int use_bias, const float *bias,
                           int use_res, const float *residual);
/* kernels/gemv.cu:2346-2397 gemv_q4_k_pair */
void or_gemv_q4k_pair(const uint8_t *wa, const uint8_t *wb, const int8_t *xq,
                      const float *xd, float *out_a, float *out_b, int n_rows,
                      int n_a, int n_b, int col_bytes, int use_bias,
                      const float *ba, const float *bb);
/* kernels/gemv.cu:2401-2436 gemv_q4_k_dual */
void or_gemv_q4k_dual(const uint8_t *wa, const uint8_t *wb, const int8_t *xq,
                      const float *xd, float *out_a, float *out_b, int n_rows,
                      int n_cols, int col_bytes);
/* FFN gate+up+SiLU.  ways = 1: gemv.cu:2546-2575 gemv_q4_k_ffn_mcol
 * (x quantized in-block, full K per warp); 2: gemv.cu:2440 gemv_q4_k_ffn;
 * 4: gemv.cu:2510 _4way; 8: gemv.cu:2578 _8way.  xq/xd are the quantized x. */
void or_gemv_q4k_ffn(const uint8_t *gate, const uint8_t *up, const int8_t *xq,
                     const float *xd, float *out, int n_rows, int n_cols,
                     int col_bytes, int ways);
/* kernels/gemv.cu:2662-2707 gemv_q4_k_qkv */
void or_gemv_q4k_qkv(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv,
                     const int8_t *xq, const float *xd, float *q, float *k,
                     float *v, int n_rows, int n_q, int n_k, int n_v,
                     int col_bytes, int use_bias, const float *bq,
                     const float *bk, const float *bv);
/* kernels/gemv.cu:515-536 gemv_q6_k_compact_global (212-byte blocks) */
void or_gemv_q6k_compact_q8(const uint8_t *w, const int8_t *xq,
                            const float *xd, float *out, int n_rows,
                            int n_cols, int col_bytes, int use_bias,
                            const float *bias, int use_res,
                            const float *residual);
/* kernels/gemv.cu:2025-2054 (_4way, ways=4) / 2081-2115 (_8way, ways=8) */
void or_gemv_q6k_compact_q8_kway(const uint8_t *w, const int8_t *xq,
                                 const float *xd, float *out, int n_rows,
                                 int n_cols, int col_bytes, int ways,
                                 int use_bias, const float *bias, int use_res,
                                 const float *residual);
/* kernels/gemv.cu:1998-2020 gemv_q6_k_compact_global_splitk */
void or_gemv_q6k_compact_q8_splitk(const uint8_t *w, const int8_t *xq,
                                   const float *xd, float *partial,
                                   int n_rows, int n_cols, int col_bytes,
                                   int n_split);
/* kernels/gemv.cu:405-438 gemv_q6_k (f32 activation, 210-byte blocks) */
void or_gemv_q6k_f32(const uint8_t *w, const float *x, float *out, int n_rows,
                     int n_cols, int col_bytes, int use_bias,
                     const float *bias, int use_res, const float *residual);
/* cuda/load.rs:145-159 align_q6_decode: 210-byte -> 212-byte blocks */
void or_q6k_compact_repack(const uint8_t *raw, uint8_t *out, int n_rows,
                           int n_cols, int col_bytes);

/* fp64 truth.  rowabs (optional) receives sum |term| per column, the
 * scale against which cancellation error is judged.  block_bytes: 144 for
 * Q4_K; 210 or 212 for Q6_K.                                        */
void or_gemv_q4k_q8_f64(const uint8_t *w, const int8_t *xq, const float *xd,
                        double *out, double *rowabs, int n_rows, int n_cols,
                        int col_bytes);
void or_gemv_q6k_q8_f64(const uint8_t *w, int block_bytes, const int8_t *xq,
                        const float *xd, double *out, double *rowabs,
                        int n_rows, int n_cols, int col_bytes);
void or_gemv_q6k_f32_f64(const uint8_t *w, const float *x, double *out,
                         double *rowabs, int n_rows, int n_cols,
                         int col_bytes);

/* ------------------------------------------------ Q8_0 / Q5_0 GEMVs
 * Q8_0 block (32 values, 34 bytes): f16 d | int8 qs[32]; value t = d*qs[t].
 * Q5_0 block (32 values, 22 bytes): f16 d | u32 qh | u8 qs[16]; value t < 16
 * = d*((qs[t] & 15 | bit t of qh << 4) - 16), value 16+t = d*((qs[t] >> 4 |
 * bit 16+t of qh << 4) - 16).  A column holds floor(n_rows/32) blocks.    */

/* kernels/gemv.cu:1558-1582 dot_q8_0_col_q8_range + :1614-1635
 * gemv_q8_0_global: per lane acc += dw*xd[bi]*(float)isum over blocks
 * bi = lane, lane+32, ..., warp_sum, then [+res] [+bias]. */
void or_gemv_q8_0_q8(const uint8_t *w, const int8_t *xq, const float *xd,
                     float *out, int n_rows, int n_cols, int col_bytes,
                     int use_bias, const float *bias, int use_res,
                     const float *residual);
/* kernels/gemv.cu:1725-1749 gemv_q8_0_global_splitk: partial[s*n_cols+j]
 * over blocks [floor(nb*s/n_split), floor(nb*(s+1)/n_split)). */
void or_gemv_q8_0_q8_splitk(const uint8_t *w, const int8_t *xq,
                            const float *xd, float *partial, int n_rows,
                            int n_cols, int col_bytes, int n_split);
/* kernels/gemv.cu:2117-2156 gemv_q8_0_splitk: f32 activation, fp32
 * products acc += (float)qs[t]*d*x[t] in block order per lane. */
void or_gemv_q8_0_f32_splitk(const uint8_t *w, const float *x, float *partial,
                             int n_rows, int n_cols, int col_bytes,
                             int n_split);
/* kernels/gemv.cu:1751-1804 gemv_q5_0 (and :2268-2296 dot_q5_0_col_xs):
 * acc += (float)(q-16)*d*x[t] for t = 0..15, low then high half. */
void or_gemv_q5_0_f32(const uint8_t *w, const float *x, float *out,
                      int n_rows, int n_cols, int col_bytes, int use_bias,
                      const float *bias, int use_res, const float *residual);
/* kernels/gemv.cu:2158-2200 gemv_q5_0_splitk */
void or_gemv_q5_0_f32_splitk(const uint8_t *w, const float *x, float *partial,
                             int n_rows, int n_cols, int col_bytes,
                             int n_split);
/* Exact int32 sums of each Q8_0 block against the Q8 activation:
 * sums[j*nb + bi]. */
void or_q8_0_block_sums(const uint8_t *w, const int8_t *xq, int32_t *sums,
                        int n_rows, int n_cols, int col_bytes);
/* fp64 truth of the three products (rowabs as above). */
void or_gemv_q8_0_q8_f64(const uint8_t *w, const int8_t *xq, const float *xd,
                         double *out, double *rowabs, int n_rows, int n_cols,
                         int col_bytes);
void or_gemv_q8_0_f32_f64(const uint8_t *w, const float *x, double *out,
                          double *rowabs, int n_rows, int n_cols,
                          int col_bytes);
void or_gemv_q5_0_f32_f64(const uint8_t *w, const float *x, double *out,
                          double *rowabs, int n_rows, int n_cols,
                          int col_bytes);

/* ------------------------------------------------------ prefill GEMMs
 * out[t*n_cols + j] = sum_i W[i][j] * x[t*n_rows + i] for n_tok tokens.
 * kernels/gemm.cu:6-67 gemm_q4_k and :69-121 gemm_q6_k (32 threads per
 * column): each super-block is dequantized to f32 as
 * common.cu:64-84 dequant_q4_k_block_smem (d*sc*q - dmin*m) or :164-186
 * dequant_q6_k_block_smem (d*sc*q); thread l accumulates wv*x over values
 * l, l+32, ... of every super-block in order; warp_sum.  The Q6_K weights
 * are raw 210-byte blocks.                                            */
void or_gemm_q4k(const uint8_t *w, const float *x, float *out, int n_rows,
                 int n_cols, int col_bytes, int n_tok);
void or_gemm_q6k(const uint8_t *w, const float *x, float *out, int n_rows,
                 int n_cols, int col_bytes, int n_tok);

/* kernels/attn/fast_v2.cu:12-103 attn_fast_v2 (128 threads): causal
 * attention of n_q queries at positions pos0 .. pos0+n_q-1 over the f16
 * cache; 64-key tiles, online softmax with expf, block_max / block_sum
 * halving trees (ops.cu:507-529), out = acc / max(l, 1e-20).  q and out
 * are [n_q][n_head*head_dim].                                        */
void or_attn_prefill(const float *q, const uint16_t *k_cache,
                     const uint16_t *v_cache, float *out, int n_head, int n_kv,
                     int head_dim, int pos0, int n_q, float scale);

/* kernels/attn/flash.cu:16-116 attn_flash_partial (n_q = 1, 128 threads) */
void or_flash_partial(const float *q, const uint16_t *k_cache,
                      const uint16_t *v_cache, float *partial, int n_head,
                      int n_kv, int head_dim, int pos0, int n_split,
                      float scale);
/* kernels/attn/flash.cu:222-255 attn_flash_reduce */
void or_flash_reduce(const float *partial, float *out, int n_head,
                     int head_dim, int n_split);
/* Textbook softmax attention in fp64 over the same f16 cache. */
void or_attn_f64(const float *q, const uint16_t *k_cache,
                 const uint16_t *v_cache, double *out, int n_head, int n_kv,
                 int head_dim, int seq_len, float scale);

/* Decode-step glue.
 * kernels/embed.cu:51-131: dequantize row `token` (block_bytes 144 = Q4_K,
 * 210 = raw Q6_K) into out[n_rows]. */
void or_embed_row(const uint8_t *table, int block_bytes, int token, int n_rows,
                  int col_bytes, float *out);
/* kernels/ops.cu:4-34 with 256 threads: strided per-thread sums of squares,
 * halving tree, scale = 1/sqrt(ss/n + eps), out = (x*scale)*w. */
void or_rms_norm(const float *x, const float *w, float *out, int n, float eps);
/* kernels/ops.cu:348-371 rope_neox_f32 (one token, all heads). */
void or_rope_neox(float *x, int n_heads, int head_dim, int pos, float theta);
/* kernels/ops.cu:471-486 copy_kv_f16: f16 bits with round-half-up. */
void or_f32_to_f16_array(const float *src, uint16_t *dst, int n);
/* Largest value, lowest index among exact ties. */
int or_argmax(const float *x, int n);
void or_flash_partial_mt(const float *q, const uint16_t *k_cache,
                         const uint16_t *v_cache, float *partial, int n_head,
                         int n_kv, int head_dim, int pos0, int n_split,
                         float scale, int nthreads);

/* CPU baseline: or_gemv_q4k_q8 / or_gemv_q6k_compact_q8_kway with the
 * output columns partitioned over nthreads POSIX threads.           */
void or_gemv_q4k_q8_mt(const uint8_t *w, const int8_t *xq, const float *xd,
                       float *out, int n_rows, int n_cols, int col_bytes,
                       int nthreads);
void or_gemv_q4k_ffn_mt(const uint8_t *gate, const uint8_t *up,
                        const int8_t *xq, const float *xd, float *out,
                        int n_rows, int n_cols, int col_bytes, int nthreads);
void or_gemv_q6k_compact_q8_kway_mt(const uint8_t *w, const int8_t *xq,
                                    const float *xd, float *out, int n_rows,
                                    int n_cols, int col_bytes, int ways,
                                    int nthreads);

#ifdef __cplusplus
}
#endif
#endif
