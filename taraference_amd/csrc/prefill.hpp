// Internal prefill entry points used by the decode runtime (model.cpp):
// the GEMM with an accumulate option and the batched glue of the n_tok-row
// forward (prefill.hip).
#pragma once
#include <stdint.h>

#include "taraference_hip.h"

// out[t][j] (+)= sum_k W[k][j] x[t][k]; q6: raw 210-byte Q6_K, else Q4_K.
// ws (ws_floats, 16-byte aligned, may be null) lets a GEMM with few output
// tiles split K into slices summed in a fixed order afterwards;
// kGemmWsFloats covers every shape.
int tf_gemm_kq(bool q6, const uint8_t* w, const float* x, float* out, int n_rows, int n_cols,
               int col_bytes, int n_tok, int accumulate, tf_stream_t stream, float* ws,
               size_t ws_floats);
// split-K workspace that serves any shape: n_split * n_tok * n_cols with
// n_split = ceil(512 / tiles) with tiles < 384 of 32 x 128 outputs needs at
// most 896 tiles of slices; a larger split (the tuning override) is clamped
// to what fits.
static const size_t kGemmWsFloats = (size_t)1152 * 32 * 128;
int tf_attn_prefill_any(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                        float* out, int n_head, int n_kv, int head_dim, int pos0,
                        const int* pos0_dev, int n_q, float scale, tf_stream_t stream);
// out[t] = embedding row of tokens_dev[t] (Q4_K 144 or Q6_K 210 blocks).
int tf_pf_embed(const uint8_t* table, int block_bytes, const int* tokens_dev, float* out,
                int n_rows, int col_bytes, int n_tok, tf_stream_t stream);
// out[t] = rmsnorm(x[t]) * w for n_tok rows of n.
int tf_pf_rms_norm(const float* x, const float* w, float* out, int n, int n_tok, float eps,
                   tf_stream_t stream);
// biases, NeoX RoPE of q and k at positions pos0 + t, k and v appended to
// the f16 caches at rows pos0 + t.
int tf_pf_qkv_post(float* q, float* k, float* v, const float* bq, const float* bk,
                   const float* bv, uint16_t* k_cache, uint16_t* v_cache, int n_head, int n_kv,
                   int head_dim, int pos0, int n_tok, float theta, tf_stream_t stream);
// g = silu(g) * u over n values.
int tf_pf_silu_mul(float* g, const float* u, long long n, tf_stream_t stream);
