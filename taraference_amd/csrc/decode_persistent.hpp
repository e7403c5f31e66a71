// Host/device interface of the persistent decode-step kernel
// (decode_persistent.hip): one launch runs a whole batch-1 decode step,
// embedding to argmax, for a dense Qwen2-style Q4_K_M model.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Per-layer weights as the kernel reads them (a device-resident table).
struct TfPLayer {
    const float* attn_norm;
    const float* ffn_norm;
    const uint8_t* wq;    // Q4_K
    const uint8_t* wk;    // Q4_K
    const uint8_t* wv;    // Q6_K (raw 210-byte blocks, f32 activation) or Q4_K
    const uint8_t* wo;    // Q4_K
    const uint8_t* gate;  // Q4_K
    const uint8_t* up;    // Q4_K
    const uint8_t* down;  // Q4_K, or the compact 212-byte Q6_K copy
    const float* bq;      // optional biases (nullptr = none)
    const float* bk;
    const float* bv;
    uint16_t* k_cache;  // f16 [max_seq][n_kv * head_dim]
    uint16_t* v_cache;
    int v_q6k, down_q6k;
    int cb_qk, cb_v, cb_o, cb_gu, cb_down;  // column bytes
};

// Control words (u32 index into TfPArgs::bar), each on its own 128-byte
// line: the launch generation (tags of the flagged vectors derive from it),
// the abort flag and the lm_head completion ticket.
#define TF_BAR_GEN 0
#define TF_BAR_ABORT 32
#define TF_BAR_DONE 64
#define TF_BAR_WORDS 96
#define TF_P_MAX_WG 1024
// Most split-KV workgroups per kv head (the partial buffer's capacity).
#define TF_P_MAX_SPLIT 64

struct TfPArgs {
    const TfPLayer* layers;
    int n_layer;
    int E, F, H, KV, HD;
    float theta, eps, scale;
    const uint8_t* embd;
    int embd_cb, embd_q6k;
    const uint8_t* head;  // compact Q6_K lm_head
    int head_cb, n_vocab;
    const float* out_norm;
    // Stage outputs as flagged words (value bits | tag << 32), each double-
    // buffered by layer parity: fx [4][E] (residual after wo: parity 0, 1;
    // after down: parity 0, 1), fq [2][H * HD] roped query, fkv [2][KV][2][HD]
    // the new K and V rows (f16 bits), fo [2][H * HD] attention output,
    // fh [2][F] silu(gate) * up.
    // nbuf = 2 double-buffers them by layer parity; nbuf = n_layer keeps
    // one copy per layer (fx [2][n_layer][E]: after wo, then after down),
    // so every layer's vectors can be read back after the step.
    unsigned long long *fx, *fq, *fkv, *fo, *fh;
    int nbuf;
    float* logits;  // [n_vocab]
    // split-KV partials (m, l, O[HD]) as tagged words [KV][G][TF_P_MAX_SPLIT][2 + HD]
    unsigned long long* fpart;
    unsigned long long* amax;  // TF_ARGMAX_SLOTS argmax keys
    unsigned* bar;             // TF_BAR_WORDS barrier words
    int* err;                  // nonzero after a barrier time-out
    // optional stage timeline: trace[(k * n_wg + wg) * 4 + {0, 1, 2, 3}] =
    // the 100 MHz realtime counter when stage k of workgroup wg starts (its
    // wait returned), arrives, has staged its activation and has finished
    // its compute (before draining its stores); nullptr = off
    unsigned long long* trace;
    // decode state.  A host-mode launch takes the token and position as
    // kernel arguments and writes the argmax to *argmax; otherwise the device
    // state advances as a replayed graph step needs (position, step, token,
    // forced prompt, token log).
    int* argmax;
    int *pos, *step, *token;
    const int *forced, *nforced;
    int* log;
    // optional Q8 record (nullptr = off): for layer slot li (0 .. n_layer;
    // slot n_layer is the lm_head input) and site s (0 QKV input, 1 attention
    // output, 2 gate/up input, 3 silu(gate) * up), the f32 values one of the
    // kernel's quantizers consumed and the Q8 it produced, at offset
    // (4 li + s) q8n (q8x, q8q) and (4 li + s) q8n / 32 (q8d).  Each value
    // is written by the workgroup that quantized it (workgroup 0 for the
    // inputs every workgroup quantizes alike).
    float* q8x;
    int8_t* q8q;
    float* q8d;
    int q8n;
};

// True when the kernel has an instantiation for this shape.
bool tf_decode_persistent_supported(int n_layer, int E, int F, int H, int KV, int HD);
// LDS bytes and grid the kernel launches with (0 grid = not launchable).
int tf_decode_persistent_grid(const TfPArgs& a, int* lds_bytes);
// Enqueue one decode step on `stream`.  `dev` is a device copy of `a` (the
// kernel reads its tables from there); host_mode != 0 decodes `token` at
// `pos`, otherwise the device state is used and advanced.
// long_ctx selects the instantiation that runs long-context attention on
// the matrix cores (valid at every position; tf_decode_persistent_long_ctx
// says where it pays).
int tf_decode_persistent_launch(const TfPArgs& a, const TfPArgs* dev, int host_mode, int token,
                                int pos, hipStream_t stream, bool long_ctx);
// True when the attention of a step at `pos` runs as one head group with
// one wave per query head on a `grid`-workgroup launch (the regime of the
// matrix-core tiles).
bool tf_decode_persistent_long_ctx(const TfPArgs& a, int grid, int pos);
