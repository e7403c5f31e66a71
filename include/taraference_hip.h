/*
 * taraference_hip.h -- C ABI of the MI355X (gfx950) batch-1 decode hot path.
 *
 * Drop-in replacement for the launch layer behind taraference's Rust
 * operator API (agkomyint/taraference v0.5.3, crates/core/src/cuda/).  Each
 * entry point replaces one NVRTC kernel symbol that the Rust side binds in
 * types.rs:302-475 and launches from matmul.rs / layer.rs.  It keeps that
 * kernel's argument list and meaning, appends the stream, and chooses the
 * launch geometry internally.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers owned by the caller.  The kernel entry
 *     points never allocate device memory; only tf_model_create (the decode
 *     runtime, at load time) allocates its workspace and KV cache.
 *   - Weights use the reference layout.  n_rows = K is the input length and
 *     n_cols = N is the number of outputs.  Output column j occupies
 *     col_bytes bytes at w + j*col_bytes and holds floor(n_rows/256)
 *     super-blocks: Q4_K blocks are 144 B and must be 16-byte aligned;
 *     compact Q6_K blocks are 212 B (cuda/load.rs:145-159) and raw Q6_K
 *     blocks are 210 B.  As in the reference, a K tail that is not a whole
 *     super-block is ignored (kernels/gemv.cu:397,484).
 *   - The Q8 activation is int8 q8[K] plus f32 d8[K/32]
 *     (kernels/gemv.cu:43-65).
 *   - use_res selects the residual: 0 = none, 1 = out[j] = acc + residual[j],
 *     2 = out[j] += acc in place.  The bias is added after the residual
 *     (kernels/gemv.cu:367-373).
 *   - The return value is a hipError_t: 0 on success, hipErrorInvalidValue
 *     (1) for a shape or pointer that the kernel cannot serve, or the launch
 *     error.  Launches are asynchronous on `stream` (a hipStream_t; NULL is
 *     the default stream).
 */
#ifndef TARAFERENCE_HIP_H
#define TARAFERENCE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *tf_stream_t; /* hipStream_t */

/* Number of 64-bit key slots of an argmax key buffer (fused lm_head argmax):
 * the caller allocates TF_ARGMAX_SLOTS zeroed unsigned long longs once. */
#define TF_ARGMAX_SLOTS 1024

/* Library version (major*10000 + minor*100 + patch). */
int tf_version(void);

/* Number of entries in tf_exported_symbols(). */
int tf_exported_symbol_count(void);
/* Name of the i-th C-ABI entry point (used by tests that check exports). */
const char *tf_exported_symbol(int i);

/* ------------------------------------------------------------ Q8 quantize */

/* kernels/gemv.cu:43 quantize_q8_global; host cuda/matmul.rs:47
 * quantize_q8.  x f32[n_rows] -> q8 int8[n_rows], d8 f32[n_rows/32].
 * n_rows % 32 == 0. */
int tf_quantize_q8(const float *x, int8_t *q8, float *d8, int n_rows,
                   tf_stream_t stream);

/* ------------------------------------------------------- Q4_K x Q8 GEMVs */

/* kernels/gemv.cu:469 gemv_q4_k_global (matmul.rs:142-302 single pass):
 * out[j] = dot(Q4_K column j, Q8 x) [+res] [+bias]. */
int tf_gemv_q4k_q8(const uint8_t *w, const int8_t *xq, const float *xd,
                   float *out, int n_rows, int n_cols, int col_bytes,
                   int use_bias, const float *bias, int use_res,
                   const float *residual, tf_stream_t stream);

/* kernels/gemv.cu:1877 gemv_q4_k_global_splitk (matmul.rs:225-283):
 * partial[s*n_cols + j] = dot over super-blocks
 * [floor(nb*s/n_split), floor(nb*(s+1)/n_split)). 1 <= n_split <= 8. */
int tf_gemv_q4k_q8_splitk(const uint8_t *w, const int8_t *xq,
                          const float *xd, float *partial, int n_rows,
                          int n_cols, int col_bytes, int n_split,
                          tf_stream_t stream);

/* kernels/gemv.cu:2243 gemv_splitk_reduce: out[j] = sum_s partial[s][j]
 * [+res] [+bias]. */
int tf_gemv_splitk_reduce(const float *partial, float *out, int n_cols,
                          int n_split, int use_bias, const float *bias,
                          int use_res, const float *residual,
                          tf_stream_t stream);

/* kernels/gemv.cu:2346 gemv_q4_k_pair (matmul.rs:727-784 try_gemv_q4_pair):
 * out_a = W_a x (+ba), out_b = W_b x (+bb), one launch, shared Q8 x. */
int tf_gemv_q4k_pair(const uint8_t *wa, const uint8_t *wb, const int8_t *xq,
                     const float *xd, float *out_a, float *out_b, int n_rows,
                     int n_a, int n_b, int col_bytes, int use_bias,
                     const float *ba, const float *bb, tf_stream_t stream);

/* kernels/gemv.cu:2401 gemv_q4_k_dual (matmul.rs:582-624 try_gemv_q4_dual):
 * equal-width pair without bias. */
int tf_gemv_q4k_dual(const uint8_t *wa, const uint8_t *wb, const int8_t *xq,
                     const float *xd, float *out_a, float *out_b, int n_rows,
                     int n_cols, int col_bytes, tf_stream_t stream);

/* kernels/gemv.cu:2440 gemv_q4_k_ffn (and _4way :2510, _8way :2578):
 * out[j] = silu(gate_j . x) * (up_j . x) with x pre-quantized. */
int tf_gemv_q4k_ffn(const uint8_t *gate, const uint8_t *up, const int8_t *xq,
                    const float *xd, float *out, int n_rows, int n_cols,
                    int col_bytes, tf_stream_t stream);

/* kernels/gemv.cu:377 gemv_q4_k (matmul.rs:346-412 gemv_baseline): f32
 * activation, quantized to Q8 inside every workgroup (bit-identically to
 * tf_quantize_q8), then the Q4_K x Q8 dot. */
int tf_gemv_q4k_f32(const uint8_t *w, const float *x, float *out, int n_rows,
                    int n_cols, int col_bytes, int use_bias, const float *bias,
                    int use_res, const float *residual, tf_stream_t stream);

/* kernels/gemv.cu:2546 gemv_q4_k_ffn_mcol (matmul.rs:680-697): as
 * tf_gemv_q4k_ffn but x is f32 and is quantized to Q8 inside every
 * workgroup (in LDS), bit-identically to tf_quantize_q8. */
int tf_gemv_q4k_ffn_f32(const uint8_t *gate, const uint8_t *up,
                        const float *x, float *out, int n_rows, int n_cols,
                        int col_bytes, tf_stream_t stream);

/* kernels/gemv.cu:2662 gemv_q4_k_qkv (matmul.rs:962-1002 try_gemv_qkv):
 * Q, K and V projections in one launch; all three Q4_K with the same K. */
int tf_gemv_q4k_qkv(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv,
                    const int8_t *xq, const float *xd, float *q, float *k,
                    float *v, int n_rows, int n_q, int n_k, int n_v,
                    int col_bytes, int use_bias, const float *bq,
                    const float *bk, const float *bv, tf_stream_t stream);

/* ------------------------------------------------------- Q6_K GEMVs */

/* kernels/gemv.cu:515 gemv_q6_k_compact_global (matmul.rs:165-169,285-300):
 * compact 212-byte Q6_K blocks x Q8 (the lm_head path). */
int tf_gemv_q6k_compact_q8(const uint8_t *w, const int8_t *xq,
                           const float *xd, float *out, int n_rows,
                           int n_cols, int col_bytes, int use_bias,
                           const float *bias, int use_res,
                           const float *residual, tf_stream_t stream);

/* kernels/gemv.cu:2081 gemv_q6_k_compact_global_8way and :2025 _4way
 * (matmul.rs:196-223): the tall Q6_K ffn_down.  The in-block split-K merge
 * and the residual/bias epilogue are fused; no partial buffer. */
int tf_gemv_q6k_down_splitk(const uint8_t *w, const int8_t *xq,
                            const float *xd, float *out, int n_rows,
                            int n_cols, int col_bytes, int use_bias,
                            const float *bias, int use_res,
                            const float *residual, tf_stream_t stream);

/* kernels/gemv.cu:1998 gemv_q6_k_compact_global_splitk: partial[s][j]
 * over super-block split s, combined by tf_gemv_splitk_reduce. */
int tf_gemv_q6k_compact_q8_splitk(const uint8_t *w, const int8_t *xq,
                                  const float *xd, float *partial,
                                  int n_rows, int n_cols, int col_bytes,
                                  int n_split, tf_stream_t stream);

/* kernels/gemv.cu:405 gemv_q6_k (matmul.rs:346-412 gemv_baseline): raw
 * 210-byte Q6_K blocks times an f32 activation, fp32 arithmetic (attn_v). */
int tf_gemv_q6k_f32(const uint8_t *w, const float *x, float *out, int n_rows,
                    int n_cols, int col_bytes, int use_bias,
                    const float *bias, int use_res, const float *residual,
                    tf_stream_t stream);

/* cuda/load.rs:145-159 align_q6_decode, on the device: copy raw 210-byte
 * blocks to 212-byte compact blocks (two zero pad bytes).
 * dst holds n_cols * floor(n_rows/256) * 212 bytes. */
int tf_q6k_compact_repack(const uint8_t *raw, uint8_t *dst, int n_rows,
                          int n_cols, int col_bytes, tf_stream_t stream);

/* ------------------------------------------------ Q8_0 / Q5_0 GEMVs
 * 32-value block formats (the tensors of width 896, not a multiple of 256,
 * in Qwen2.5-0.5B Q4_K_M files).  Q8_0 block = f16 d | int8 qs[32] (34 B);
 * Q5_0 block = f16 d | u32 qh | u8 qs[16] (22 B), value = d * (code - 16).
 * n_rows % 32 == 0; column j holds n_rows/32 blocks at w + j*col_bytes;
 * weights 2-byte aligned.  Q8_0 x Q8 uses a faster pair layout when
 * n_rows/32 is even and the columns are 4-byte aligned.  The f32
 * activations are 16-byte aligned (8 for the Q8_0 entry points that
 * quantize); the f32 formats stage at most 16384 rows.            */

/* kernels/gemv.cu:1614 gemv_q8_0_global (matmul.rs:142-302, 305-330):
 * out[j] = sum over blocks of dw * xd * int8 dot [+res] [+bias]. */
int tf_gemv_q8_0_q8(const uint8_t *w, const int8_t *xq, const float *xd,
                    float *out, int n_rows, int n_cols, int col_bytes,
                    int use_bias, const float *bias, int use_res,
                    const float *residual, tf_stream_t stream);

/* kernels/gemv.cu:1585 gemv_q8_0 (matmul.rs:346-412 gemv_baseline): as
 * tf_gemv_q8_0_q8 with x f32, quantized in LDS bit-identically to
 * tf_quantize_q8. */
int tf_gemv_q8_0_f32(const uint8_t *w, const float *x, float *out, int n_rows,
                     int n_cols, int col_bytes, int use_bias, const float *bias,
                     int use_res, const float *residual, tf_stream_t stream);

/* kernels/gemv.cu:1725 gemv_q8_0_global_splitk (matmul.rs:225-283):
 * partial[s*n_cols + j] over blocks [floor(nb*s/n_split),
 * floor(nb*(s+1)/n_split)), combined by tf_gemv_splitk_reduce.
 * 1 <= n_split <= 64. */
int tf_gemv_q8_0_q8_splitk(const uint8_t *w, const int8_t *xq,
                           const float *xd, float *partial, int n_rows,
                           int n_cols, int col_bytes, int n_split,
                           tf_stream_t stream);

/* kernels/gemv.cu:2117 gemv_q8_0_splitk (matmul.rs:416-500 gemv_splitk):
 * f32 activation, fp32 products d * qs[t] * x[t]; partials as above. */
int tf_gemv_q8_0_f32_splitk(const uint8_t *w, const float *x, float *partial,
                            int n_rows, int n_cols, int col_bytes,
                            int n_split, tf_stream_t stream);

/* kernels/gemv.cu:1751 gemv_q5_0 (matmul.rs:346-412): fp32 products
 * d * (code - 16) * x [+res] [+bias]. */
int tf_gemv_q5_0_f32(const uint8_t *w, const float *x, float *out, int n_rows,
                     int n_cols, int col_bytes, int use_bias, const float *bias,
                     int use_res, const float *residual, tf_stream_t stream);

/* kernels/gemv.cu:2158 gemv_q5_0_splitk (matmul.rs:416-500). */
int tf_gemv_q5_0_f32_splitk(const uint8_t *w, const float *x, float *partial,
                            int n_rows, int n_cols, int col_bytes,
                            int n_split, tf_stream_t stream);

/* kernels/gemv.cu:2298 gemv_q5_0_qk (matmul.rs:786-840): q = Wq x (+bq),
 * k = Wk x (+bk) in one launch (also gate+up); both Q5_0, same K. */
int tf_gemv_q5_0_qk(const uint8_t *wq, const uint8_t *wk, const float *x,
                    float *q, float *k, int n_rows, int n_q, int n_k,
                    int col_bytes, int use_bias, const float *bq,
                    const float *bk, tf_stream_t stream);

/* kernels/gemv.cu:2710 gemv_q5_0_qkv (matmul.rs:1087-1130). */
int tf_gemv_q5_0_qkv(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv,
                     const float *x, float *q, float *k, float *v, int n_rows,
                     int n_q, int n_k, int n_v, int col_bytes, int use_bias,
                     const float *bq, const float *bk, const float *bv,
                     tf_stream_t stream);

/* kernels/gemv.cu:2766 gemv_q8_0_qkv (matmul.rs:1003-1080): x f32,
 * quantized in LDS as tf_quantize_q8, then as tf_gemv_q8_0_q8. */
int tf_gemv_q8_0_qkv(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv,
                     const float *x, float *q, float *k, float *v, int n_rows,
                     int n_q, int n_k, int n_v, int col_bytes, int use_bias,
                     const float *bq, const float *bk, const float *bv,
                     tf_stream_t stream);

/* ------------------------------------------------------------- prefill
 * n_tok > 1 (the prompt).  x, q and out are row-major per token:
 * x[t*n_rows + k], out[t*n_cols + j], q/out of attention [t][n_head*hd].  */

/* kernels/gemm.cu:6 gemm_q4_k (matmul.rs:1269-1323 gemm): out[t][j] =
 * sum_k W[k][j] x[t][k], x f32, fp32 accuracy (matrix cores on exact
 * integer weights and a three-part bf16 split of x; scales in fp32).
 * n_rows % 4 == 0 (floor(n_rows/256) super-blocks are used, as the
 * reference), x and out 16-byte aligned, w and col_bytes 4-byte aligned. */
int tf_gemm_q4k_f32(const uint8_t *w, const float *x, float *out, int n_rows,
                    int n_cols, int col_bytes, int n_tok, tf_stream_t stream);

/* kernels/gemm.cu:69 gemm_q6_k: the same over raw 210-byte Q6_K blocks
 * (2-byte aligned). */
int tf_gemm_q6k_f32(const uint8_t *w, const float *x, float *out, int n_rows,
                    int n_cols, int col_bytes, int n_tok, tf_stream_t stream);

/* kernels/attn/fast_v2.cu:12 attn_fast_v2 (layer.rs prefill attention):
 * causal attention of n_q queries at positions pos0 .. pos0+n_q-1 over the
 * f16 cache [seq][n_kv*head_dim] (rows 0 .. pos0+n_q-1 written),
 * out = softmax(q k^T * scale) v per head, GQA head h -> kv h/(n_head/n_kv).
 * head_dim 64, 128 or 256; q/out 16-byte aligned. */
int tf_attn_prefill(const float *q, const uint16_t *k_cache,
                    const uint16_t *v_cache, float *out, int n_head, int n_kv,
                    int head_dim, int pos0, int n_q, float scale,
                    tf_stream_t stream);

/* kernels/attn/fast_v2.cu:103 attn_fast_v2_d: pos0 read from device memory
 * (graph-capturable). */
int tf_attn_prefill_d(const float *q, const uint16_t *k_cache,
                      const uint16_t *v_cache, float *out, int n_head, int n_kv,
                      int head_dim, const int *pos0_dev, int n_q, float scale,
                      tf_stream_t stream);

/* ---------------------------------------------------- split-KV flash decode */

/* kernels/attn/flash.cu:16 attn_flash_partial (layer.rs:2040-2103), n_q = 1.
 * q f32[n_head*head_dim]; k_cache/v_cache f16 bits [seq][n_kv*head_dim];
 * attends positions 0..pos0.  The sequence is split into n_split chunks of
 * ceil((pos0+1)/n_split) tokens and partial[(h*n_split+s)*(2+head_dim)]
 * receives (m, l, O[head_dim]) with O not yet divided by l.  An empty chunk
 * writes (-1e30, 0, 0...).  n_head % n_kv == 0, head_dim % 4 == 0,
 * head_dim <= 256, 1 <= n_split <= 1024. */
int tf_flash_decode_partial(const float *q, const uint16_t *k_cache,
                            const uint16_t *v_cache, float *partial,
                            int n_head, int n_kv, int head_dim, int pos0,
                            int n_q, int n_split, float scale,
                            tf_stream_t stream);

/* kernels/attn/flash.cu:119 attn_flash_partial_d: pos0 read from device
 * memory so that a captured HIP graph stays valid as the position moves. */
int tf_flash_decode_partial_d(const float *q, const uint16_t *k_cache,
                              const uint16_t *v_cache, float *partial,
                              int n_head, int n_kv, int head_dim,
                              const int *pos0_dev, int n_q, int n_split,
                              float scale, tf_stream_t stream);

/* kernels/attn/flash.cu:222 attn_flash_reduce: log-sum-exp merge,
 * out[h*head_dim+d] = sum_s e^(m_s-M) O_s[d] / max(sum_s e^(m_s-M) l_s, 1e-20). */
int tf_flash_decode_reduce(const float *partial, float *out, int n_head,
                           int head_dim, int n_split, int n_q,
                           tf_stream_t stream);

/* kernels/attn/flash.cu:16/:119 + :222 as one call (layer.rs:2040-2121):
 * split-KV partials, then the log-sum-exp merge (a second kernel); when
 * q8/d8 are non-NULL the merged output is also quantized to Q8 (quantize_q8
 * of the wo GEMV input, matmul.rs:191).  pos0_dev non-NULL reads the position
 * from device memory (graph capture).  counters: reserved, not used (may be
 * NULL).  partial as for tf_flash_decode_partial. */
int tf_flash_decode(const float *q, const uint16_t *k_cache,
                    const uint16_t *v_cache, float *partial, unsigned *counters,
                    float *out, int8_t *q8, float *d8, int n_head, int n_kv,
                    int head_dim, int pos0, const int *pos0_dev, int n_split,
                    float scale, tf_stream_t stream);
/* flash.cu:222 attn_flash_reduce + quantize_q8 + gemv.cu:469
 * gemv_q4_k_global (the attention output projection wo, layer.rs:2104-2119
 * then matmul.rs:142): every workgroup merges the split-KV partials of all
 * n_head heads (log-sum-exp, split order), quantizes the merged row to Q8 in
 * LDS and runs the Q4_K GEMV on it; out[j] = dot (use_res 0) or out[j] +=
 * dot (use_res 2).  n_head <= 32, n_head*head_dim % 256 == 0 and <= 4096,
 * n_split <= 64, n_head*(n_split+1) <= 2048.  attn_out / attn_q8 / attn_d8
 * (all NULL or all set) receive the merged row and its Q8. */
int tf_gemv_q4k_flash_out(const uint8_t *w, const float *partial, int n_head,
                          int head_dim, int n_split, float *out, int n_cols,
                          int col_bytes, int use_res, float *attn_out,
                          int8_t *attn_q8, float *attn_d8, tf_stream_t stream);
/* No counterpart in the reference: tf_flash_decode for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The split partials live in a
 * static device array of this library (one per GPU, held until the process
 * ends): n_head * n_split * (2 + head_dim) <= 2^20 floats, else
 * hipErrorInvalidValue.  Allocates nothing and enqueues nothing but the
 * flash kernels, so it may be captured into a HIP graph from its first call.
 * Calls that overlap on one GPU share that array and race. */
int tf_flash_decode_noalloc(const float *q, const uint16_t *k_cache,
                            const uint16_t *v_cache, float *out, int8_t *q8,
                            float *d8, int n_head, int n_kv, int head_dim,
                            int pos0, const int *pos0_dev, int n_split,
                            float scale, tf_stream_t stream);
/* No counterpart in the reference (a parity check): the persistent decode
 * step's in-kernel quantizers applied to x[n] (n % 32 == 0), writing the Q8
 * of quantize_q8_global (kernels/gemv.cu:43-65): variant 0 = the eight-lane
 * staging of its RMSNorm outputs, 1 = the sixteen-lane quantization of the
 * attention output and of silu(gate)*up. */
int tf_decode_step_quantize_q8(const float *x, int n, int variant, int8_t *q,
                               float *d, tf_stream_t stream);
/* No counterpart in the reference (a measurement aid for bench.py): reads
 * n_bytes (a multiple of 16) at src with 16-byte loads, `depth` (4, 8 or 16)
 * in flight per thread, on blocks_per_cu (1..8) x CUs workgroups of 512
 * threads (contiguous != 0: each workgroup reads its own contiguous run,
 * else the threads interleave over the whole buffer), and writes one word
 * per workgroup to sink (blocks_per_cu x CUs words).  The plain
 * streaming-read rate the GEMVs are priced against. */
int tf_stream_read_probe(const void *src, long long n_bytes, uint32_t *sink,
                         int blocks_per_cu, int depth, int contiguous,
                         tf_stream_t stream);
/* Partition count this library recommends for a context of max_seq tokens
 * (a multiple of 8; 8 for short contexts).  The reference fixes 8
 * (cuda/decode.rs:38-41); on MI355X long contexts need more partitions to
 * occupy 256 CUs.  The caller sizes partial[] as
 * n_head * n_split * (2 + head_dim) floats. */
int tf_flash_decode_n_split(int n_kv, int max_seq);

/* ------------------------------------------------------- decode-step glue */

/* kernels/embed.cu:51-131 embed_q{4,6}_k_one[_d] and embed_q{5,8}_0_one[_d]:
 * dequantize row `token` (or *token_dev when token_dev != NULL) of a Q4_K
 * (block_bytes 144), raw Q6_K (210), Q8_0 (34) or Q5_0 (22) table into
 * out[n_rows]. */
int tf_embed_row(const uint8_t *table, int block_bytes, float *out, int token,
                 const int *token_dev, int n_rows, int col_bytes,
                 tf_stream_t stream);
/* kernels/ops.cu:4-34 rms_norm_f32 (one row): out = x * rsqrt(mean x^2 + eps) * w */
int tf_rms_norm(const float *x, const float *w, float *out, int n, float eps,
                tf_stream_t stream);
/* kernels/ops.cu:348-398 rope_neox_f32[_d]: rotate (i, i+hd/2) of every head
 * by pos * theta^(-2i/hd); pos read from pos_dev when non-NULL. */
int tf_rope_neox(float *x, int n_heads, int head_dim, int pos,
                 const int *pos_dev, float theta, tf_stream_t stream);
/* kernels/ops.cu:471-504 copy_kv_f16[_d]: cache[pos*stride + i] =
 * f16(src[i]) with the reference's round-half-up conversion. */
int tf_copy_kv_f16(const float *src, uint16_t *cache, int pos,
                   const int *pos_dev, int stride, tf_stream_t stream);
/* kernels/ops.cu:573-599 argmax_f32 (one 256-thread block, layer.rs:2248-2255):
 * *out_idx = the reference's winner.  NaN and values <= -1e30 never win
 * (index 0 if nothing beats -1e30); among exact ties (-0 == +0) the index
 * whose residue i mod 256, bit-reversed over 8 bits, is smallest wins, then
 * the smallest i of that residue. */
int tf_argmax(const float *x, int n, int *out_idx, tf_stream_t stream);

/* ------------------------------------------------------ fused decode kernels */
/* Each fuses a chain of reference kernels that the reference launches back
 * to back in its decode step; every stage keeps the arithmetic of its
 * unfused counterpart (normalization and Q8 bytes are bit-identical, GEMV
 * sums differ only in fp32 summation order). */

/* layer.rs:171-645: rms_norm_f32 + quantize_q8 + gemv_q4_k_pair (Q, K, bias)
 * + V projection (gemv_q6_k f32 activation when v_type is Q6_K, Q4_K x Q8
 * otherwise; bias) + rope_neox_f32 on Q and K + copy_kv_f16 of K and V at
 * position pos (or *pos_dev).  x is the residual stream (n_embd floats);
 * norm_w may be NULL (no normalization).  q_out receives the rotated Q; the
 * f16 K/V rows go to k_cache/v_cache [seq][n_kv*head_dim]. */
int tf_fused_norm_qkv_rope_kv(const float *x, const float *norm_w, float eps,
                              const uint8_t *wq, const uint8_t *wk,
                              const uint8_t *wv, int v_type, const float *bq,
                              const float *bk, const float *bv, int n_embd,
                              int n_head, int n_kv, int head_dim,
                              int col_bytes_qk, int col_bytes_v, float *q_out,
                              uint16_t *k_cache, uint16_t *v_cache, int pos,
                              const int *pos_dev, float theta,
                              tf_stream_t stream);
/* The same as tf_fused_norm_qkv_rope_kv with the activation already
 * normalized and quantized (tf_norm_quant): xq/xd its Q8, xb its f32 values
 * (read by the Q6_K V projection; may be NULL when v_type is Q4_K). */
int tf_fused_qkv_rope_kv(const int8_t *xq, const float *xd, const float *xb,
                         const uint8_t *wq, const uint8_t *wk, const uint8_t *wv,
                         int v_type, const float *bq, const float *bk,
                         const float *bv, int n_embd, int n_head, int n_kv,
                         int head_dim, int col_bytes_qk, int col_bytes_v,
                         float *q_out, uint16_t *k_cache, uint16_t *v_cache,
                         int pos, const int *pos_dev, float theta,
                         tf_stream_t stream);
/* ops.cu:4-34 rms_norm_f32 + gemv.cu:43-65 quantize_q8_global, one launch:
 * xb = x * rsqrt(mean x^2 + eps) * w and its Q8 (q8[n], d8[n/32]);
 * n % 128 == 0, n <= 8192; x, w, xb 8-byte aligned. */
int tf_norm_quant(const float *x, const float *w, float eps, float *xb,
                  int8_t *q8, float *d8, int n, tf_stream_t stream);
/* flash.cu:222 attn_flash_reduce + quantize_q8 of the attention output
 * (layer.rs:2104-2119 then matmul.rs:191): also writes q8[n_head*head_dim]
 * and d8[n_head*head_dim/32]; head_dim % 64 == 0. */
int tf_flash_decode_reduce_q8(const float *partial, float *out, int8_t *q8,
                              float *d8, int n_head, int head_dim,
                              int n_split, tf_stream_t stream);
/* layer.rs:2181-2257 with a pre-quantized activation:
 * gemv_q6_k_compact_global (logits) + argmax into amax_key[TF_ARGMAX_SLOTS] (see
 * tf_gemv_q6k_head_argmax). */
int tf_gemv_q6k_q8_argmax(const uint8_t *w, const int8_t *xq, const float *xd,
                          float *logits, int n_rows, int n_cols, int col_bytes,
                          unsigned long long *amax_key, tf_stream_t stream);
/* layer.rs:1220-1386: rms_norm_f32 (x * norm_w) + gemv_q4_k_ffn_mcol. */
int tf_gemv_q4k_ffn_norm(const uint8_t *gate, const uint8_t *up,
                         const float *x, const float *norm_w, float eps,
                         float *out, int n_rows, int n_cols, int col_bytes,
                         tf_stream_t stream);
/* matmul.rs:191-223: quantize_q8 + the compact Q6_K GEMV (f32 activation
 * quantized inside every workgroup); use_res 0 or 2 (in place). */
int tf_gemv_q6k_compact_f32(const uint8_t *w, const float *x, float *out,
                            int n_rows, int n_cols, int col_bytes, int use_res,
                            tf_stream_t stream);
/* layer.rs:2158-2257: rms_norm_f32 (when norm_w != NULL) + quantize_q8 +
 * gemv_q6_k_compact_global (logits) + argmax_f32.  The argmax is
 * accumulated as 64-bit keys into amax_key[TF_ARGMAX_SLOTS], which must
 * hold zeros at launch; read it with tf_argmax_key_finalize, which also
 * resets every slot to 0. */
int tf_gemv_q6k_head_argmax(const uint8_t *w, const float *x,
                            const float *norm_w, float eps, float *logits,
                            int n_rows, int n_cols, int col_bytes,
                            unsigned long long *amax_key, tf_stream_t stream);
/* *out_idx = index of the largest key in amax_key[TF_ARGMAX_SLOTS] (largest
 * logit, ties and NaN as tf_argmax); every slot is reset to 0. */
int tf_argmax_key_finalize(unsigned long long *amax_key, int *out_idx,
                           tf_stream_t stream);

/* ----------------------------------------------------- decode-step runtime */
/* C++ restatement of the reference model runtime for dense Qwen2-style
 * models (cuda/forward.rs:42-407, cuda/layer.rs:99-709,1210-1456,2125-2259,
 * cuda/model.rs:522-570): one greedy decode step per call, optionally
 * replayed from a captured HIP graph with the position and token in device
 * memory.  Weights are caller-owned device buffers. */

#define TF_TYPE_Q4_K 12 /* GGML type ids */
#define TF_TYPE_Q6_K 14
#define TF_TYPE_Q5_0 6  /* K = 896 tensors of Qwen2.5-0.5B files (path 0 only) */
#define TF_TYPE_Q8_0 8

/* cuda/types.rs:212-225 GpuMat: data = GGUF bytes; compact = 212-byte Q6_K
 * repack (NULL for Q4_K). */
typedef struct tf_mat {
    const uint8_t *data;
    const uint8_t *compact;
    int type;
    int n_rows;
    int n_cols;
    int col_bytes;
    int compact_col_bytes;
} tf_mat;

typedef struct tf_layer {
    const float *attn_norm;
    tf_mat wq, wk, wv;
    const float *bq, *bk, *bv; /* NULL when the model has no QKV bias */
    tf_mat wo;
    const float *ffn_norm;
    tf_mat gate, up, down;
} tf_layer;

typedef struct tf_model_config {
    int n_layer, n_embd, n_ff, n_head, n_kv, head_dim, n_vocab, max_seq;
    float rope_theta, rms_eps;
} tf_model_config;

typedef struct tf_model tf_model;

/* cuda/load.rs:166 + model.rs:522: bind weights, allocate workspace and the
 * f16 KV cache [n_layer][max_seq][n_kv*head_dim] (K and V). token_embd is
 * the embedding table; output is the lm_head (may be the same tensor). */
int tf_model_create(const tf_model_config *cfg, const tf_layer *layers,
                    const tf_mat *token_embd, const tf_mat *output,
                    const float *output_norm, tf_model **out);
void tf_model_destroy(tf_model *m);
/* cuda/forward.rs:42 forward_greedy for one token at position pos: runs the
 * eager kernel sequence, leaves logits on the device, *next_token set on the
 * host (blocks on the stream). */
int tf_model_forward(tf_model *m, int token, int pos, int *next_token,
                     tf_stream_t stream);
/* Runs n_forced + n_gen - 1 decode steps (n_forced if n_gen == 0) from
 * position pos0 with the position,
 * token and outputs kept in device memory (forward.rs:73-264; replayed from
 * a captured HIP graph when use_graph).  Step i < n_forced consumes
 * forced[i] (a prompt fed through the decode path); later steps consume the
 * previous argmax.  tokens[i] (i < n_gen) receives the argmax of step
 * n_forced - 1 + i, i.e. the greedy continuation.  The stream is
 * synchronized once, at the end. */
int tf_model_generate(tf_model *m, const int *forced, int n_forced, int pos0,
                      int n_gen, int *tokens, int use_graph, tf_stream_t stream);
/* cuda/forward.rs:42-71 forward_greedy for n_tok > 1 (the prompt): the
 * tokens at positions pos0 .. pos0+n_tok-1 go through the n_tok-row forward
 * in chunks of 256 (the prefill GEMMs and attention, f32 activations, as the
 * reference's prefill), their K/V rows are written to the cache, and
 * *next_token receives the argmax of the last token's logits (left on the
 * device as after a decode step).  Continue with tf_model_generate(forced =
 * {*next_token}, pos0 + n_tok, ...).  Weights must be Q4_K / Q6_K.  Blocks on
 * the stream. */
int tf_model_prefill(tf_model *m, const int *tokens, int n_tok, int pos0,
                     int *next_token, tf_stream_t stream);
/* Select the kernel sequence of a step (all compute the same step):
 *   0  the reference's sequence through the operator API (cuda/layer.rs
 *      order, one launch per reference kernel);
 *   1  fused kernels, each activation normalized / quantized once by its
 *      own launch (nine launches per layer);
 *   2  fused kernels with the normalization / quantization and
 *      the attention merge in the consuming GEMV's prologue (five launches
 *      per layer);
 *   3  as 2, with h quantized by its own launch before a Q8 ffn_down
 *      (the default where path 4 does not apply);
 *   4  the whole step (embedding to argmax) in one persistent launch, one
 *      workgroup per CU, stages exchanging tagged vectors (no barriers); returns
 *      hipErrorNotSupported for a model shape or weight mix it has no
 *      instantiation for (the default where it applies).
 * Changing the path drops the captured graph. */
int tf_model_set_path(tf_model *m, int path);
/* The decode path in use (the default chosen at creation, or the last
 * tf_model_set_path); -1 for a null handle. */
int tf_model_get_path(const tf_model *m);
/* Device pointer of the last logits (n_vocab floats) and of the f16 K/V
 * cache of layer li. */
const float *tf_model_logits(const tf_model *m);
/* Inspection of the persistent step (path 4); no counterpart in the
 * reference.  on != 0 before the first path-4 step makes the step keep one
 * copy of every stage vector per layer instead of two alternating ones
 * (hipErrorNotSupported once the step's buffers exist with the other
 * setting).  tf_model_stage_vector then returns layer li's vector of `kind`
 * after a step, as 64-bit words whose low half is the value bits and high
 * half a tag: 0 = residual after the attention output projection (f32,
 * n_embd words), 1 = residual after the FFN down projection (f32, n_embd),
 * 2 = roped query (f32, n_head*head_dim), 4 = attention output and
 * 5 = silu(gate)*up, both as Q8 in groups of 9 words per 32 values (8
 * words of four int8 in value order, then the f32 scale).  NULL when not
 * kept. */
int tf_model_keep_stage_vectors(tf_model *m, int on);
const unsigned long long *tf_model_stage_vector(const tf_model *m, int kind,
                                                int li);
/* No counterpart in the reference (a parity check of the persistent step):
 * with the stage vectors kept, the step also records, for every quantizer
 * it runs, the f32 values quantized and the Q8 produced.  site 0 = the
 * normalized input of the QKV GEMVs (li = n_layer: of the lm_head), 1 = the
 * merged attention output, 2 = the normalized input of gate/up, 3 =
 * silu(gate)*up; part 0 = f32 values, 1 = int8 q, 2 = f32 d per 32 values.
 * Device pointer; NULL when not kept or out of range. */
const void *tf_model_q8_record(const tf_model *m, int site, int li, int part);
uint16_t *tf_model_k_cache(const tf_model *m, int li);
uint16_t *tf_model_v_cache(const tf_model *m, int li);

/* ------------------------------------------------------------- GGUF reader */
/* crates/gguf/src/reader.rs:29-169 GgufFile::open and its accessors: the file
 * is memory-mapped read-only; tensor bytes are pointers into the mapping (host
 * memory) for the caller to upload (cuda/load.rs:178-271).  Versions 2 and 3;
 * the checks of the reference (magic, version, counts <= 1e6, strings
 * <= 64 MiB and valid UTF-8, arrays <= 1e7 items, n_dims <= 4, known ggml
 * types, every tensor inside the file) map to the TF_GGUF_ERR_* codes. */
#define TF_GGUF_ERR_ARG 1          /* hipErrorInvalidValue: bad argument */
#define TF_GGUF_ERR_IO 1001        /* GgufError::Io */
#define TF_GGUF_ERR_MAGIC 1002     /* GgufError::BadMagic */
#define TF_GGUF_ERR_VERSION 1003   /* GgufError::UnsupportedVersion */
#define TF_GGUF_ERR_EOF 1004       /* GgufError::UnexpectedEof */
#define TF_GGUF_ERR_MALFORMED 1005 /* GgufError::Malformed */
#define TF_GGUF_ERR_TENSOR_TYPE 1006 /* GgufError::UnknownTensorType */
#define TF_GGUF_ERR_VALUE_TYPE 1007  /* GgufError::UnknownValueType */
#define TF_GGUF_ERR_UTF8 1008      /* GgufError::InvalidUtf8 */
#define TF_GGUF_ERR_NOT_FOUND 1009 /* no such key / tensor (Option::None) */
#define TF_GGUF_ERR_TYPE 1010      /* the value does not convert (Option::None) */

/* value.rs:8-23 ValueType ids */
#define TF_GGUF_U8 0
#define TF_GGUF_I8 1
#define TF_GGUF_U16 2
#define TF_GGUF_I16 3
#define TF_GGUF_U32 4
#define TF_GGUF_I32 5
#define TF_GGUF_F32 6
#define TF_GGUF_BOOL 7
#define TF_GGUF_STRING 8
#define TF_GGUF_ARRAY 9
#define TF_GGUF_U64 10
#define TF_GGUF_I64 11
#define TF_GGUF_F64 12

typedef struct tf_gguf tf_gguf;

/* types.rs:193-201 GgufTensorInfo (+ its data slice, reader.rs:201-205);
 * dims past n_dims read 1; name lives as long as the handle. */
typedef struct tf_gguf_tensor {
    const char *name;
    int type;
    int n_dims;
    uint64_t dims[4];
    uint64_t offset; /* relative to the data section */
    uint64_t nbytes; /* types.rs:178-189 nbytes of the element count */
    const uint8_t *data;
} tf_gguf_tensor;

int tf_gguf_open(const char *path, tf_gguf **out);
void tf_gguf_close(tf_gguf *g);
uint32_t tf_gguf_version(const tf_gguf *g);
/* reader.rs:143-149: header end aligned to general.alignment (default 32) */
uint64_t tf_gguf_data_offset(const tf_gguf *g);
uint64_t tf_gguf_file_size(const tf_gguf *g);
int64_t tf_gguf_n_tensors(const tf_gguf *g);
int tf_gguf_tensor_at(const tf_gguf *g, int64_t i, tf_gguf_tensor *out);
/* reader.rs:196-198 tensor(name) */
int tf_gguf_find_tensor(const tf_gguf *g, const char *name, tf_gguf_tensor *out);
/* metadata: the value type id of key, -1 if absent */
int tf_gguf_meta_type(const tf_gguf *g, const char *key);
/* value.rs:72-106 as_u32 / as_u64 / as_f32 / as_str / as_bool (the same
 * conversions; TF_GGUF_ERR_TYPE where those return None) */
int tf_gguf_meta_u32(const tf_gguf *g, const char *key, uint32_t *out);
int tf_gguf_meta_u64(const tf_gguf *g, const char *key, uint64_t *out);
int tf_gguf_meta_f32(const tf_gguf *g, const char *key, float *out);
int tf_gguf_meta_str(const tf_gguf *g, const char *key, const char **s, uint64_t *len);
int tf_gguf_meta_bool(const tf_gguf *g, const char *key, int *out);
/* No reference counterpart (its Value enum is matched directly): any signed
 * or unsigned integer as int64, any float as f64, array item type and length,
 * and array items as string or as number. */
int tf_gguf_meta_i64(const tf_gguf *g, const char *key, int64_t *out);
int tf_gguf_meta_f64(const tf_gguf *g, const char *key, double *out);
int tf_gguf_meta_array(const tf_gguf *g, const char *key, int *item_type, uint64_t *n);
int tf_gguf_meta_array_str(const tf_gguf *g, const char *key, uint64_t i, const char **s,
                           uint64_t *len);
int tf_gguf_meta_array_f64(const tf_gguf *g, const char *key, uint64_t i, double *out);
/* types.rs:109-180 ggml type table: block size, bytes per block (0 for an
 * unknown type) and the bytes of n elements. */
int tf_ggml_block_size(int type);
int tf_ggml_type_size(int type);
uint64_t tf_ggml_nbytes(int type, uint64_t n_elements);
/* config.rs:107-175 ModelConfig::from_gguf, the dense-decoder fields: the
 * {arch}.embedding_length, block_count, attention.head_count,
 * feed_forward_length keys are required; head_count_kv defaults to
 * head_count, key_length to embedding_length / head_count (value_length must
 * equal it), vocab_size to token_embd.weight dims[1], rope.freq_base to 1e4
 * for llama and 1e6 otherwise, attention.layer_norm_rms_epsilon to 1e-6.
 * max_seq is the caller's KV capacity. */
int tf_gguf_model_config(const tf_gguf *g, int max_seq, tf_model_config *cfg);

/* ------------------------------------------------------- integer diagnostics */
/* No reference counterpart: these expose the exact integer stage of the GEMV
 * kernels (the same device code) so that the int32 sums can be checked
 * bit-exactly.  For column j, super-block bi and sub-block g:
 *   Q4_K: dots[(j*nb+bi)*8+g] = sum q4*q8, sums[...] = sum q8 (32 values)
 *   Q6_K: dots[(j*nb+bi)*16+g] = sum (q6-32)*q8 (16 values)          */
int tf_q4k_block_dots(const uint8_t *w, const int8_t *xq, int32_t *dots,
                      int32_t *sums, int n_rows, int n_cols, int col_bytes,
                      tf_stream_t stream);
int tf_q6k_block_dots(const uint8_t *w, int block_bytes, const int8_t *xq,
                      int32_t *dots, int n_rows, int n_cols, int col_bytes,
                      tf_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* TARAFERENCE_HIP_H */
