// Decode-step runtime for dense Qwen2-style Q4_K_M models: the C++
// restatement of the reference model runtime (cuda/forward.rs,
// cuda/layer.rs, cuda/model.rs, cuda/kv.rs) for batch-1 greedy decode.
//
// Per token (layer.rs:99-709 attn_block, :1210-1456 ffn_block_dense,
// :2125-2259 logits_from_last):
//   x = embed(token)
//   per layer: xb = rmsnorm(x) * attn_norm
//              q, k = Wq xb + bq, Wk xb + bk        (Q4_K pair on Q8 xb)
//              v = Wv xb + bv                        (f32 activation GEMV)
//              rope(q), rope(k); K/V -> f16 cache at pos
//              xb = flash_decode(q, K[0..pos], V[0..pos])
//              x += Wo q8(xb)
//              xb = rmsnorm(x) * ffn_norm
//              hb = silu(Wg q8(xb)) * (Wu q8(xb))
//              x += Wdown q8(hb)
//   logits = lm_head q8(rmsnorm(x) * output_norm); next = argmax(logits)
// The graph path keeps the position, the current token, the forced prompt
// and the generated tokens in device memory (forward.rs:73-264), so a
// captured step can be replayed back to back without host round trips.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <algorithm>
#include <cstdlib>
#include <memory>
#include <new>
#include <vector>

#include "argmax_key.hpp"
#include "decode_persistent.hpp"
#include "op_api.hpp"
#include "prefill.hpp"
#include "taraference_hip.h"

namespace {

using tf::GemvResidual;
using tf::GpuMat;

GpuMat to_mat(const tf_mat& m) {
    GpuMat g;
    g.data = m.data;
    g.compact_data = m.compact;
    g.n_rows = (size_t)m.n_rows;
    g.n_cols = (size_t)m.n_cols;
    g.col_bytes = (size_t)m.col_bytes;
    g.compact_col_bytes = (size_t)m.compact_col_bytes;
    g.wtype = m.type == TF_TYPE_Q6_K   ? tf::WType::Q6K
              : m.type == TF_TYPE_Q5_0 ? tf::WType::Q5_0
              : m.type == TF_TYPE_Q8_0 ? tf::WType::Q8_0
                                       : tf::WType::Q4K;
    return g;
}

struct Layer {
    const float* attn_norm;
    GpuMat wq, wk, wv, wo, gate, up, down;
    const float *bq, *bk, *bv;
    const float* ffn_norm;
};

// Advance the device-side decode state after one step: log the argmax,
// select the next input token (forced prompt token or the argmax) and move
// to the next position.
__global__ void tf_decode_advance_kernel(int* pos, int* step, int* token, const int* argmax,
                                         unsigned long long* amax_key, const int* forced,
                                         const int* n_forced, int* log) {
    int next = 0;
    if (amax_key) next = tf_argmax_key_index(tf_argmax_slots_take(amax_key));  // fused head
    if (threadIdx.x != 0) return;
    const int s = *step;
    if (!amax_key) next = *argmax;
    log[s] = next;
    *token = (s + 1 < *n_forced) ? forced[s + 1] : next;
    *pos += 1;
    *step = s + 1;
}

template <class T>
T* dev_alloc(size_t n) {
    void* p = nullptr;
    if (hipMalloc(&p, n * sizeof(T) + 256) != hipSuccess) throw std::bad_alloc();
    return static_cast<T*>(p);
}

}  // namespace

struct tf_model {
    tf_model_config cfg{};
    std::vector<Layer> layers;
    GpuMat token_embd, output;
    const float* output_norm = nullptr;
    int embd_block_bytes = 210;
    tf::FlashDims fd{};

    // workspace (cuda/load.rs:502-607)
    float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *hb = nullptr;
    float* hb2 = nullptr;  // up projection when gate/up are not fused
    float *logits = nullptr, *flash_partial = nullptr, *gemv_partial = nullptr;
    int8_t* q8_x = nullptr;
    float* q8_d = nullptr;
    size_t partial_stride = 0;
    std::vector<uint16_t*> kc, vc;
    // device decode state
    int *d_pos = nullptr, *d_step = nullptr, *d_token = nullptr, *d_argmax = nullptr;
    unsigned long long* d_amax_key = nullptr;
    // 0: the reference operator sequence (step); 1: fused, each activation
    // normalized and quantized once by its own kernel; 2: fused, the
    // normalization / quantization / attention merge runs in the consuming
    // GEMV's prologue; 3: as 2 but h is quantized by its own kernel;
    // 4: the whole step in one persistent launch (decode_persistent.hip).
    // Default: 4 when persistent_ok(), else 3 (set in tf_model_create).
    int path = 3;
    // persistent-step state (allocated on first use of path 4)
    TfPLayer* d_players = nullptr;
    unsigned* d_bar = nullptr;
    int* d_perr = nullptr;
    unsigned long long* p_part = nullptr;
    size_t p_part_words = 0;
    unsigned long long* p_flags = nullptr;  // the flagged stage vectors
    bool p_keep = false;  // one copy of them per layer (tf_model_keep_stage_vectors)
    size_t p_flag_words = 0;
    // the Q8 record of the step's quantizers (TfPArgs::q8x), kept with the
    // stage vectors
    float *p_q8x = nullptr, *p_q8d = nullptr;
    int8_t* p_q8q = nullptr;
    int p_q8n = 0;
    // diagnostic stage timeline of the persistent step: when the environment
    // names a file in TF_P_TRACE, the last step of each run() is written there
    unsigned long long* d_trace = nullptr;
    size_t trace_words = 0;
    TfPArgs pargs{};
    TfPArgs* d_pargs = nullptr;
    unsigned* d_flash_cnt = nullptr;  // per-kv-head tickets of tf_flash_decode
    int *d_forced = nullptr, *d_nforced = nullptr, *d_log = nullptr;
    // prefill workspace (n_tok-row activations of one chunk), allocated on
    // the first prefill
    float *pf_x = nullptr, *pf_xb = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr,
          *pf_att = nullptr, *pf_g = nullptr, *pf_u = nullptr, *pf_ws = nullptr;
    int* pf_tok = nullptr;
    std::vector<void*> allocs;

    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    // kGraphSteps consecutive steps in one graph (fewer graph launches per token)
    static constexpr int kGraphSteps = 8;
    hipGraph_t graph_n = nullptr;
    hipGraphExec_t graph_exec_n = nullptr;
    hipStream_t capture_stream = nullptr;

    template <class T>
    T* alloc(size_t n) {
        T* p = dev_alloc<T>(n);
        allocs.push_back(p);
        return p;
    }

    ~tf_model() {
        drop_graph();
        if (capture_stream) (void)hipStreamDestroy(capture_stream);
        for (void* p : allocs) (void)hipFree(p);
    }

    // One decode step.  pos_dev == nullptr: host position `pos` and host
    // token `token`; otherwise both are read from device memory.
    void step(hipStream_t s, int token, int pos, bool device_state) {
        const tf_model_config& c = cfg;
        const int* pos_dev = device_state ? d_pos : nullptr;
        const int* tok_dev = device_state ? d_token : nullptr;
        tf::check(tf_embed_row(token_embd.data, embd_block_bytes, x, token, tok_dev, c.n_embd,
                               (int)token_embd.col_bytes, s),
                  "embed");
        const int stride = c.n_kv * c.head_dim;
        for (size_t li = 0; li < layers.size(); li++) {
            const Layer& L = layers[li];
            // ---- attention block
            tf::check(tf_rms_norm(x, L.attn_norm, xb, c.n_embd, c.rms_eps, s), "rms_norm");
            if (!tf::try_gemv_qkv(s, L.wq, L.wk, L.wv, xb, q, k, v, L.bq, L.bk, L.bv, q8_x, q8_d)) {
                if (tf::try_gemv_pair(s, L.wq, L.wk, xb, q, k, L.bq, L.bk, q8_x, q8_d) ||
                    tf::try_gemv_q5_dual(s, L.wq, L.wk, xb, q, k, L.bq, L.bk)) {
                    tf::gemv(s, L.wv, xb, v, L.bv, GemvResidual::none(), gemv_partial,
                             partial_stride);
                } else {
                    tf::gemv(s, L.wq, xb, q, L.bq, GemvResidual::none(), gemv_partial, partial_stride);
                    tf::gemv(s, L.wk, xb, k, L.bk, GemvResidual::none(), gemv_partial, partial_stride);
                    tf::gemv(s, L.wv, xb, v, L.bv, GemvResidual::none(), gemv_partial, partial_stride);
                }
            }
            tf::check(tf_rope_neox(q, c.n_head, c.head_dim, pos, pos_dev, c.rope_theta, s), "rope q");
            tf::check(tf_rope_neox(k, c.n_kv, c.head_dim, pos, pos_dev, c.rope_theta, s), "rope k");
            tf::check(tf_copy_kv_f16(k, kc[li], pos, pos_dev, stride, s), "copy k");
            tf::check(tf_copy_kv_f16(v, vc[li], pos, pos_dev, stride, s), "copy v");
            tf::launch_attn_flash(s, fd, q, kc[li], vc[li], flash_partial, xb, pos, pos_dev);
            if (!tf::try_gemv_global_q8(s, L.wo, xb, x, nullptr, GemvResidual::in_place(), q8_x,
                                        q8_d, gemv_partial, partial_stride))
                tf::gemv(s, L.wo, xb, x, nullptr, GemvResidual::in_place(), gemv_partial,
                         partial_stride);
            // ---- FFN block
            tf::check(tf_rms_norm(x, L.ffn_norm, xb, c.n_embd, c.rms_eps, s), "rms_norm");
            if (!tf::try_gemv_q4_ffn(s, L.gate, L.up, xb, hb, q8_x, q8_d)) {
                // layer.rs:1267-1390: gate and up (one dual launch when both
                // are Q5_0), then silu_mul
                if (!tf::try_gemv_q5_dual(s, L.gate, L.up, xb, hb, hb2, nullptr, nullptr)) {
                    tf::gemv(s, L.gate, xb, hb, nullptr, GemvResidual::none(), gemv_partial,
                             partial_stride);
                    tf::gemv(s, L.up, xb, hb2, nullptr, GemvResidual::none(), gemv_partial,
                             partial_stride);
                }
                tf::check(tf_pf_silu_mul(hb, hb2, c.n_ff, reinterpret_cast<tf_stream_t>(s)),
                          "silu_mul");
            }
            if (!tf::try_gemv_global_q8(s, L.down, hb, x, nullptr, GemvResidual::in_place(), q8_x,
                                        q8_d, gemv_partial, partial_stride))
                tf::gemv(s, L.down, hb, x, nullptr, GemvResidual::in_place(), gemv_partial,
                         partial_stride);
        }
        // ---- logits + argmax
        tf::check(tf_rms_norm(x, output_norm, xb, c.n_embd, c.rms_eps, s), "rms_norm");
        if (!tf::try_gemv_global_q8(s, output, xb, logits, nullptr, GemvResidual::none(), q8_x,
                                    q8_d, gemv_partial, partial_stride))
            tf::gemv(s, output, xb, logits, nullptr, GemvResidual::none(), gemv_partial,
                     partial_stride);
        tf::check(tf_argmax(logits, c.n_vocab, d_argmax, s), "argmax");
        if (device_state) {
            hipLaunchKernelGGL(tf_decode_advance_kernel, dim3(1), dim3(256), 0, s, d_pos, d_step,
                               d_token, d_argmax, nullptr, d_forced, d_nforced, d_log);
            tf::check((int)hipGetLastError(), "advance");
        }
    }

    // The same step with fused kernels: each activation is normalized and
    // quantized once (tf_norm_quant, or the flash reduce for the attention
    // output), QKV + RoPE + KV append run in one GEMV launch, and the head
    // carries the argmax: nine launches per layer (path 1).  With `prologue`
    // (paths 2 and 3) the RMSNorm + Q8 run in the staging of the QKV and
    // gate/up kernels and the split merge + Q8 in the staging of wo: six
    // launches per layer with the Q8 down (path 3), five with the f32 down.
    void step_fused(hipStream_t s, int token, int pos, bool device_state, bool prologue,
                    bool q8_down) {
        const tf_model_config& c = cfg;
        const int* pos_dev = device_state ? d_pos : nullptr;
        const int* tok_dev = device_state ? d_token : nullptr;
        tf::check(tf_embed_row(token_embd.data, embd_block_bytes, x, token, tok_dev, c.n_embd,
                               (int)token_embd.col_bytes, s),
                  "embed");
        for (size_t li = 0; li < layers.size(); li++) {
            const Layer& L = layers[li];
            if (L.wq.wtype != tf::WType::Q4K || L.wk.wtype != tf::WType::Q4K ||
                L.wq.col_bytes != L.wk.col_bytes || L.gate.wtype != tf::WType::Q4K ||
                L.up.wtype != tf::WType::Q4K)
                throw tf::HipError(1, "fused path needs Q4_K q/k/gate/up");
            const int v_type = L.wv.wtype == tf::WType::Q6K ? TF_TYPE_Q6_K : TF_TYPE_Q4_K;
            if (prologue) {
                tf::check(tf_fused_norm_qkv_rope_kv(
                              x, L.attn_norm, c.rms_eps, L.wq.data, L.wk.data, L.wv.data, v_type,
                              L.bq, L.bk, L.bv, c.n_embd, c.n_head, c.n_kv, c.head_dim,
                              (int)L.wq.col_bytes, (int)L.wv.col_bytes, q, kc[li], vc[li], pos,
                              pos_dev, c.rope_theta, s),
                          "norm+qkv");
            } else {
                tf::check(tf_norm_quant(x, L.attn_norm, c.rms_eps, xb, q8_x, q8_d, c.n_embd, s),
                          "norm_quant");
                tf::check(tf_fused_qkv_rope_kv(q8_x, q8_d, xb, L.wq.data, L.wk.data, L.wv.data,
                                               v_type, L.bq, L.bk, L.bv, c.n_embd, c.n_head,
                                               c.n_kv, c.head_dim, (int)L.wq.col_bytes,
                                               (int)L.wv.col_bytes, q, kc[li], vc[li], pos,
                                               pos_dev, c.rope_theta, s),
                          "fused qkv");
            }
            const bool wo_merge = prologue && L.wo.wtype == tf::WType::Q4K && fd.n_split <= 64 &&
                                  c.n_head <= 32 &&
                                  c.n_head * (fd.n_split + 1) <= 2048 &&
                                  c.n_head * c.head_dim <= 4096 &&
                                  (c.n_head * c.head_dim) % 256 == 0;
            if (wo_merge) {
                // split-KV partials, then wo with the merge in its prologue
                if (pos_dev)
                    tf::check(tf_flash_decode_partial_d(q, kc[li], vc[li], flash_partial,
                                                        fd.n_head, fd.n_kv, fd.head_dim, pos_dev,
                                                        1, fd.n_split, fd.scale, s),
                              "flash partial");
                else
                    tf::check(tf_flash_decode_partial(q, kc[li], vc[li], flash_partial, fd.n_head,
                                                      fd.n_kv, fd.head_dim, pos, 1, fd.n_split,
                                                      fd.scale, s),
                              "flash partial");
                tf::check(tf_gemv_q4k_flash_out(L.wo.data, flash_partial, fd.n_head, fd.head_dim,
                                                fd.n_split, x, (int)L.wo.n_cols,
                                                (int)L.wo.col_bytes, 2, nullptr, nullptr,
                                                nullptr, s),
                          "merge+wo");
            } else {
                // attention with its merge and the Q8 of the merged output
                tf::check(tf_flash_decode(q, kc[li], vc[li], flash_partial, d_flash_cnt, xb, q8_x,
                                          q8_d, fd.n_head, fd.n_kv, fd.head_dim, pos, pos_dev,
                                          fd.n_split, fd.scale, s),
                          "flash");
                gemv_q8_inplace(s, L.wo);
            }
            if (prologue) {
                tf::check(tf_gemv_q4k_ffn_norm(L.gate.data, L.up.data, x, L.ffn_norm, c.rms_eps,
                                               hb, c.n_embd, c.n_ff, (int)L.gate.col_bytes, s),
                          "norm+ffn");
                if (q8_down) {
                    tf::check(tf_quantize_q8(hb, q8_x, q8_d, c.n_ff, s), "quantize h");
                    gemv_q8_inplace(s, L.down);
                } else {
                    gemv_f32_inplace(s, L.down, hb);
                }
            } else {
                tf::check(tf_norm_quant(x, L.ffn_norm, c.rms_eps, xb, q8_x, q8_d, c.n_embd, s),
                          "norm_quant");
                tf::check(tf_gemv_q4k_ffn(L.gate.data, L.up.data, q8_x, q8_d, hb, c.n_embd,
                                          c.n_ff, (int)L.gate.col_bytes, s),
                          "ffn");
                tf::check(tf_quantize_q8(hb, q8_x, q8_d, c.n_ff, s), "quantize h");
                gemv_q8_inplace(s, L.down);
            }
        }
        const bool keyed = output.wtype == tf::WType::Q6K && output.compact_data;
        if (keyed && prologue) {
            tf::check(tf_gemv_q6k_head_argmax(output.compact_data, x, output_norm, c.rms_eps,
                                              logits, (int)output.n_rows, (int)output.n_cols,
                                              (int)output.compact_col_bytes, d_amax_key, s),
                      "norm+head");
            if (!device_state)
                tf::check(tf_argmax_key_finalize(d_amax_key, d_argmax, s), "argmax");
        } else if (keyed) {
            tf::check(tf_norm_quant(x, output_norm, c.rms_eps, xb, q8_x, q8_d, c.n_embd, s),
                      "norm_quant");
            tf::check(tf_gemv_q6k_q8_argmax(output.compact_data, q8_x, q8_d, logits,
                                            (int)output.n_rows, (int)output.n_cols,
                                            (int)output.compact_col_bytes, d_amax_key, s),
                      "head");
            if (!device_state)
                tf::check(tf_argmax_key_finalize(d_amax_key, d_argmax, s), "argmax");
        } else {
            tf::check(tf_rms_norm(x, output_norm, xb, c.n_embd, c.rms_eps, s), "norm");
            tf::gemv(s, output, xb, logits, nullptr, GemvResidual::none(), gemv_partial,
                     partial_stride);
            tf::check(tf_argmax(logits, c.n_vocab, d_argmax, s), "argmax");
        }
        if (device_state) {
            hipLaunchKernelGGL(tf_decode_advance_kernel, dim3(1), dim3(256), 0, s, d_pos, d_step,
                               d_token, d_argmax, keyed ? d_amax_key : nullptr, d_forced,
                               d_nforced, d_log);
            tf::check((int)hipGetLastError(), "advance");
        }
    }

    // x += W a for the Q8 activation in q8_x/q8_d.
    void gemv_q8_inplace(hipStream_t s, const GpuMat& w) {
        if (w.wtype == tf::WType::Q4K)
            tf::check(tf_gemv_q4k_q8(w.data, q8_x, q8_d, x, (int)w.n_rows, (int)w.n_cols,
                                     (int)w.col_bytes, 0, nullptr, 2, nullptr, s),
                      "gemv q4k");
        else if (w.compact_data)
            tf::check(tf_gemv_q6k_down_splitk(w.compact_data, q8_x, q8_d, x, (int)w.n_rows,
                                              (int)w.n_cols, (int)w.compact_col_bytes, 0, nullptr,
                                              2, nullptr, s),
                      "gemv q6k");
        else
            throw tf::HipError(1, "Q6_K matrix without its compact copy");
    }

    // x += W a for the f32 activation a (quantized in the GEMV's prologue).
    void gemv_f32_inplace(hipStream_t s, const GpuMat& w, const float* a) {
        if (w.wtype == tf::WType::Q4K)
            tf::check(tf_gemv_q4k_f32(w.data, a, x, (int)w.n_rows, (int)w.n_cols,
                                      (int)w.col_bytes, 0, nullptr, 2, nullptr, s),
                      "gemv q4k f32");
        else if (w.compact_data)
            tf::check(tf_gemv_q6k_compact_f32(w.compact_data, a, x, (int)w.n_rows, (int)w.n_cols,
                                              (int)w.compact_col_bytes, 2, s),
                      "gemv q6k f32");
        else
            throw tf::HipError(1, "Q6_K matrix without its compact copy");
    }

    // Whether path 4 can serve this model: Q4_K q/k/wo/gate/up, Q6_K or
    // Q4_K v and down (Q6_K down and the lm_head with their compact copy), and
    // a shape the persistent kernel is instantiated for.
    // Paths 1-4 are written for the Q4_K_M K-quant placement: every matrix
    // Q4_K or Q6_K, widths multiples of 256.  Other models (Q5_0 / Q8_0
    // tensors, e.g. the 896-wide Qwen2.5-0.5B) run the reference sequence.
    bool kquant_ok() const {
        const tf_model_config& c = cfg;
        if (c.n_embd % 256 || c.n_ff % 256) return false;
        auto kq = [](const GpuMat& w) {
            return w.wtype == tf::WType::Q4K || w.wtype == tf::WType::Q6K;
        };
        if (!kq(token_embd) || !kq(output)) return false;
        for (const Layer& L : layers)
            if (!kq(L.wq) || !kq(L.wk) || !kq(L.wv) || !kq(L.wo) || !kq(L.gate) || !kq(L.up) ||
                !kq(L.down))
                return false;
        return true;
    }

    bool persistent_ok() const {
        if (!kquant_ok()) return false;
        const tf_model_config& c = cfg;
        if (!tf_decode_persistent_supported(c.n_layer, c.n_embd, c.n_ff, c.n_head, c.n_kv,
                                            c.head_dim))
            return false;
        if (output.wtype != tf::WType::Q6K || !output.compact_data) return false;
        for (const Layer& L : layers) {
            if (L.wq.wtype != tf::WType::Q4K || L.wk.wtype != tf::WType::Q4K ||
                L.wo.wtype != tf::WType::Q4K || L.gate.wtype != tf::WType::Q4K ||
                L.up.wtype != tf::WType::Q4K || L.wq.col_bytes != L.wk.col_bytes ||
                L.gate.col_bytes != L.up.col_bytes)
                return false;
            if (L.down.wtype == tf::WType::Q6K && !L.down.compact_data) return false;
        }
        return true;
    }

    void ensure_persistent() {
        if (d_players) return;
        const tf_model_config& c = cfg;
        std::vector<TfPLayer> h(layers.size());
        for (size_t i = 0; i < layers.size(); i++) {
            const Layer& L = layers[i];
            TfPLayer& p = h[i];
            p.attn_norm = L.attn_norm;
            p.ffn_norm = L.ffn_norm;
            p.wq = L.wq.data;
            p.wk = L.wk.data;
            p.wv = L.wv.data;
            p.wo = L.wo.data;
            p.gate = L.gate.data;
            p.up = L.up.data;
            p.v_q6k = L.wv.wtype == tf::WType::Q6K;
            p.down_q6k = L.down.wtype == tf::WType::Q6K;
            p.down = p.down_q6k ? L.down.compact_data : L.down.data;
            p.bq = L.bq;
            p.bk = L.bk;
            p.bv = L.bv;
            p.k_cache = kc[i];
            p.v_cache = vc[i];
            p.cb_qk = (int)L.wq.col_bytes;
            p.cb_v = (int)L.wv.col_bytes;
            p.cb_o = (int)L.wo.col_bytes;
            p.cb_gu = (int)L.gate.col_bytes;
            p.cb_down = (int)(p.down_q6k ? L.down.compact_col_bytes : L.down.col_bytes);
        }
        d_players = alloc<TfPLayer>(h.size());
        tf::check((int)hipMemcpy(d_players, h.data(), h.size() * sizeof(TfPLayer),
                                 hipMemcpyHostToDevice), "copy layer table");
        d_bar = alloc<unsigned>(TF_BAR_WORDS);
        d_perr = alloc<int>(1);
        const size_t nb = p_keep ? (size_t)c.n_layer : 2;
        p_flag_words = nb * (2 * (size_t)c.n_embd + (size_t)c.n_head * c.head_dim +
                             2 * (size_t)c.n_kv * c.head_dim + (size_t)c.n_head * c.head_dim +
                             (size_t)c.n_ff);
        p_flags = alloc<unsigned long long>(p_flag_words);
        p_part_words = (size_t)c.n_head * TF_P_MAX_SPLIT * (2 + c.head_dim);
        if (p_keep) {
            // a whole number of 32-value groups per record (the scales index off / 32)
            p_q8n = (std::max({c.n_embd, c.n_ff, c.n_head * c.head_dim}) + 31) & ~31;
            const size_t n = ((size_t)c.n_layer + 1) * 4 * (size_t)p_q8n;
            p_q8x = alloc<float>(n);
            p_q8q = alloc<int8_t>(n);
            p_q8d = alloc<float>(n / 32);
        }
        p_part = alloc<unsigned long long>(p_part_words);
        if (std::getenv("TF_P_TRACE")) {
            trace_words = (size_t)(5 * c.n_layer + 2) * TF_P_MAX_WG * 4;
            d_trace = alloc<unsigned long long>(trace_words);
        }
        fill_pargs();
        d_pargs = alloc<TfPArgs>(1);
        tf::check((int)hipMemcpy(d_pargs, &pargs, sizeof(TfPArgs), hipMemcpyHostToDevice),
                  "copy args");
        reset_persistent(nullptr);
    }

    // Zero the barrier words, merge tickets and error flag (a fresh
    // generation; also clears what an aborted launch left behind).
    void reset_persistent(hipStream_t s) {
        tf::check((int)hipMemsetAsync(d_bar, 0, TF_BAR_WORDS * sizeof(unsigned), s), "memset");
        tf::check((int)hipMemsetAsync(p_part, 0, p_part_words * sizeof(unsigned long long), s),
                  "memset");
        tf::check((int)hipMemsetAsync(d_perr, 0, sizeof(int), s), "memset");
        tf::check((int)hipMemsetAsync(p_flags, 0, p_flag_words * sizeof(unsigned long long), s),
                  "memset");
        if (!s) tf::check((int)hipDeviceSynchronize(), "sync");
    }

    // After a synchronization: a barrier time-out inside the persistent
    // kernel is reported as hipErrorLaunchTimeOut (and the state is reset).
    void check_persistent(hipStream_t s) {
        if (path != 4 || !d_perr) return;
        int e = 0;
        tf::check((int)hipMemcpy(&e, d_perr, sizeof(int), hipMemcpyDeviceToHost), "copy");
        if (e) {
            reset_persistent(s);
            tf::check((int)hipStreamSynchronize(s), "sync");
            throw tf::HipError((int)hipErrorLaunchTimeOut, "persistent step barrier time-out");
        }
    }

    // The persistent kernel's argument table (host copy in pargs, device
    // copy in d_pargs).
    void fill_pargs() {
        const tf_model_config& c = cfg;
        TfPArgs& a = pargs;
        a = TfPArgs{};
        a.layers = d_players;
        a.n_layer = c.n_layer;
        a.E = c.n_embd;
        a.F = c.n_ff;
        a.H = c.n_head;
        a.KV = c.n_kv;
        a.HD = c.head_dim;
        a.theta = c.rope_theta;
        a.eps = c.rms_eps;
        a.scale = fd.scale;
        a.embd = token_embd.data;
        a.embd_cb = (int)token_embd.col_bytes;
        a.embd_q6k = embd_block_bytes == 210;
        a.head = output.compact_data;
        a.head_cb = (int)output.compact_col_bytes;
        a.n_vocab = (int)output.n_cols;
        a.out_norm = output_norm;
        const size_t nb = p_keep ? (size_t)c.n_layer : 2;
        a.nbuf = (int)nb;
        a.fx = p_flags;
        a.fq = a.fx + 2 * nb * c.n_embd;
        a.fkv = a.fq + nb * c.n_head * c.head_dim;
        a.fo = a.fkv + 2 * nb * c.n_kv * c.head_dim;
        a.fh = a.fo + nb * c.n_head * c.head_dim;
        a.logits = logits;
        a.fpart = p_part;
        a.amax = d_amax_key;
        a.bar = d_bar;
        a.err = d_perr;
        a.trace = d_trace;
        a.q8x = p_q8x;
        a.q8q = p_q8q;
        a.q8d = p_q8d;
        a.q8n = p_q8n;
        a.argmax = d_argmax;
        a.pos = d_pos;
        a.step = d_step;
        a.token = d_token;
        a.forced = d_forced;
        a.nforced = d_nforced;
        a.log = d_log;
    }

    // the long-context instantiation of the persistent step (graph runs:
    // chosen in run() for the last position of the run)
    bool p_long = false;

    bool long_ctx(int pos) {
        ensure_persistent();
        const int grid = tf_decode_persistent_grid(pargs, nullptr);
        return tf_decode_persistent_long_ctx(pargs, grid, pos);
    }

    void step_persistent(hipStream_t s, int token, int pos, bool device_state) {
        ensure_persistent();
        const bool lc = device_state ? p_long : long_ctx(pos);
        tf::check(tf_decode_persistent_launch(pargs, d_pargs, device_state ? 0 : 1, token, pos, s,
                                              lc),
                  "persistent step");
    }

    void run_step(hipStream_t s, int token, int pos, bool device_state) {
        if (path == 0) step(s, token, pos, device_state);
        else if (path == 4) step_persistent(s, token, pos, device_state);
        else step_fused(s, token, pos, device_state, path >= 2, path == 3);
    }

    void drop_graph() {
        if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
        if (graph) (void)hipGraphDestroy(graph);
        if (graph_exec_n) (void)hipGraphExecDestroy(graph_exec_n);
        if (graph_n) (void)hipGraphDestroy(graph_n);
        graph_exec = nullptr;
        graph = nullptr;
        graph_exec_n = nullptr;
        graph_n = nullptr;
    }

    // A graph of `steps` consecutive decode steps (the state advances on the
    // device, so replaying it runs that many tokens).
    void capture_steps(int steps, hipGraph_t& g_out, hipGraphExec_t& e_out) {
        if (e_out) return;
        if (!capture_stream) tf::check((int)hipStreamCreateWithFlags(&capture_stream, hipStreamNonBlocking), "stream");
        tf::check((int)hipStreamBeginCapture(capture_stream, hipStreamCaptureModeThreadLocal), "capture");
        try {
            for (int i = 0; i < steps; i++) run_step(capture_stream, 0, 0, true);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(capture_stream, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        tf::check((int)hipStreamEndCapture(capture_stream, &g_out), "end capture");
        tf::check((int)hipGraphInstantiate(&e_out, g_out, nullptr, nullptr, 0), "instantiate");
    }

    void capture() { capture_steps(1, graph, graph_exec); }

    // Runs n_forced + max(n_gen, 1) - 1 steps from position pos0 with
    // device-resident state; tokens[i] = argmax of step n_forced - 1 + i.
    void run(hipStream_t s, const int* forced, int n_forced, int pos0, int n_gen, int* tokens,
             bool use_graph) {
        const int total = n_forced + (n_gen > 0 ? n_gen : 1) - 1;
        if (n_forced < 1 || pos0 < 0 || pos0 + total > cfg.max_seq)
            throw tf::HipError(1, "decode range outside the KV cache");
        std::vector<int> h(4);
        h[0] = pos0;
        h[1] = 0;
        h[2] = forced[0];
        h[3] = n_forced;
        tf::check((int)hipMemcpyAsync(d_forced, forced, sizeof(int) * n_forced,
                                      hipMemcpyHostToDevice, s), "copy prompt");
        tf::check((int)hipMemcpyAsync(d_pos, &h[0], sizeof(int), hipMemcpyHostToDevice, s), "copy");
        tf::check((int)hipMemcpyAsync(d_step, &h[1], sizeof(int), hipMemcpyHostToDevice, s), "copy");
        tf::check((int)hipMemcpyAsync(d_token, &h[2], sizeof(int), hipMemcpyHostToDevice, s), "copy");
        tf::check((int)hipMemcpyAsync(d_nforced, &h[3], sizeof(int), hipMemcpyHostToDevice, s), "copy");
        if (path == 4) {
            ensure_persistent();
            reset_persistent(s);
            const bool lc = long_ctx(pos0 + total - 1);
            if (lc != p_long) {  // the captured step launches the other instantiation
                p_long = lc;
                drop_graph();
            }
        }
        if (use_graph) {
            capture();
            if (total >= kGraphSteps) capture_steps(kGraphSteps, graph_n, graph_exec_n);
        }
        for (int i = 0; i < total;) {
            if (use_graph && total - i >= kGraphSteps) {
                tf::check((int)hipGraphLaunch(graph_exec_n, s), "graph launch");
                i += kGraphSteps;
            } else {
                if (use_graph) tf::check((int)hipGraphLaunch(graph_exec, s), "graph launch");
                else run_step(s, 0, 0, true);
                i++;
            }
        }
        if (n_gen > 0 && tokens)
            tf::check((int)hipMemcpyAsync(tokens, d_log + n_forced - 1, sizeof(int) * n_gen,
                                          hipMemcpyDeviceToHost, s), "copy tokens");
        tf::check((int)hipStreamSynchronize(s), "sync");
        check_persistent(s);
        if (path == 4 && d_trace) dump_trace();
    }

    // Prompt chunk size of the prefill (types.rs MAX_BATCH).
    static constexpr int kPrefillChunk = 256;

    // x[t] (+)= W xin[t] for n rows on the matrix cores (raw GGUF bytes).
    void gemm(hipStream_t s, const GpuMat& w, const float* xin, float* out, int n,
              bool accumulate) {
        tf::check(tf_gemm_kq(w.wtype == tf::WType::Q6K, w.data, xin, out, (int)w.n_rows,
                             (int)w.n_cols, (int)w.col_bytes, n, accumulate ? 1 : 0,
                             reinterpret_cast<tf_stream_t>(s), pf_ws, kGemmWsFloats),
                  "prefill gemm");
    }

    // The prompt forward of forward.rs:42-71 forward_greedy / :360-404
    // forward_chunk: chunks of up to kPrefillChunk tokens through the
    // n_tok-row layer (layer.rs attn_block / ffn_block_dense with
    // n_tok > 1: rms_norm rows, GEMMs, add_bias, rope, copy_kv, prefill
    // attention, GEMM + add for wo and down, silu_mul), K/V appended at
    // positions pos0 .. pos0+n-1; then the last row's logits and argmax
    // (logits_from_last), as the decode step computes them.
    void prefill(hipStream_t s, const int* tokens, int n, int pos0) {
        const tf_model_config& c = cfg;
        if (n < 1 || pos0 < 0 || pos0 + n > c.max_seq)
            throw tf::HipError((int)hipErrorInvalidValue, "prefill range outside the KV cache");
        if (!kquant_ok())
            throw tf::HipError((int)hipErrorNotSupported, "prefill needs Q4_K/Q6_K weights");
        const int CH = kPrefillChunk, E = c.n_embd, F = c.n_ff;
        const int kvd = c.n_kv * c.head_dim;
        if (!pf_x) {
            pf_x = alloc<float>((size_t)CH * E);
            pf_xb = alloc<float>((size_t)CH * E);
            pf_q = alloc<float>((size_t)CH * E);
            pf_att = alloc<float>((size_t)CH * E);
            pf_k = alloc<float>((size_t)CH * kvd);
            pf_v = alloc<float>((size_t)CH * kvd);
            pf_g = alloc<float>((size_t)CH * F);
            pf_u = alloc<float>((size_t)CH * F);
            pf_tok = alloc<int>(CH);
            pf_ws = alloc<float>(kGemmWsFloats);
        }
        const tf_stream_t ts = reinterpret_cast<tf_stream_t>(s);
        int last = 0;
        for (int off = 0; off < n; off += CH) {
            const int nt = n - off < CH ? n - off : CH;
            const int p0 = pos0 + off;
            tf::check((int)hipMemcpyAsync(pf_tok, tokens + off, sizeof(int) * nt,
                                          hipMemcpyHostToDevice, s), "copy tokens");
            tf::check(tf_pf_embed(token_embd.data, embd_block_bytes, pf_tok, pf_x, E,
                                  (int)token_embd.col_bytes, nt, ts), "embed");
            for (size_t li = 0; li < layers.size(); li++) {
                const Layer& L = layers[li];
                tf::check(tf_pf_rms_norm(pf_x, L.attn_norm, pf_xb, E, nt, c.rms_eps, ts), "rms");
                gemm(s, L.wq, pf_xb, pf_q, nt, false);
                gemm(s, L.wk, pf_xb, pf_k, nt, false);
                gemm(s, L.wv, pf_xb, pf_v, nt, false);
                tf::check(tf_pf_qkv_post(pf_q, pf_k, pf_v, L.bq, L.bk, L.bv, kc[li], vc[li],
                                         c.n_head, c.n_kv, c.head_dim, p0, nt, c.rope_theta, ts),
                          "qkv post");
                tf::check(tf_attn_prefill_any(pf_q, kc[li], vc[li], pf_att, c.n_head, c.n_kv,
                                              c.head_dim, p0, nullptr, nt, fd.scale, ts),
                          "prefill attention");
                gemm(s, L.wo, pf_att, pf_x, nt, true);
                tf::check(tf_pf_rms_norm(pf_x, L.ffn_norm, pf_xb, E, nt, c.rms_eps, ts), "rms");
                gemm(s, L.gate, pf_xb, pf_g, nt, false);
                gemm(s, L.up, pf_xb, pf_u, nt, false);
                tf::check(tf_pf_silu_mul(pf_g, pf_u, (long long)nt * F, ts), "silu_mul");
                gemm(s, L.down, pf_g, pf_x, nt, true);
            }
            last = nt - 1;
        }
        // logits of the last prompt token (the decode step's head)
        const float* xl = pf_x + (size_t)last * E;
        tf::check(tf_rms_norm(xl, output_norm, xb, E, c.rms_eps, s), "rms_norm");
        if (!tf::try_gemv_global_q8(s, output, xb, logits, nullptr, GemvResidual::none(), q8_x,
                                    q8_d, gemv_partial, partial_stride))
            tf::gemv(s, output, xb, logits, nullptr, GemvResidual::none(), gemv_partial,
                     partial_stride);
        tf::check(tf_argmax(logits, c.n_vocab, d_argmax, s), "argmax");
    }

    void dump_trace() {
        std::vector<unsigned long long> h(trace_words);
        tf::check((int)hipMemcpy(h.data(), d_trace, trace_words * sizeof(unsigned long long),
                                 hipMemcpyDeviceToHost), "copy trace");
        TfPArgs a{};
        a.E = cfg.n_embd;
        a.F = cfg.n_ff;
        a.H = cfg.n_head;
        a.KV = cfg.n_kv;
        a.HD = cfg.head_dim;
        const int grid = tf_decode_persistent_grid(a, nullptr);
        FILE* f = std::fopen(std::getenv("TF_P_TRACE"), "w");
        if (!f) return;
        std::fprintf(f, "%d %d\n", 5 * cfg.n_layer + 2, grid);
        for (int k = 0; k < 5 * cfg.n_layer + 2; k++) {
            for (int b = 0; b < grid; b++)
                for (int w = 0; w < 4; w++)
                    std::fprintf(f, "%llu ", h[((size_t)k * grid + b) * 4 + w]);
            std::fprintf(f, "\n");
        }
        std::fclose(f);
    }
};

extern "C" int tf_model_create(const tf_model_config* cfg, const tf_layer* layers,
                               const tf_mat* token_embd, const tf_mat* output,
                               const float* output_norm, tf_model** out) {
    if (!cfg || !layers || !token_embd || !output || !output_norm || !out) return (int)hipErrorInvalidValue;
    const tf_model_config& c = *cfg;
    if (c.n_layer <= 0 || c.n_embd % 32 || c.n_ff % 32 || c.n_head <= 0 || c.n_kv <= 0 ||
        c.n_head % c.n_kv || c.n_head * c.head_dim != c.n_embd || c.max_seq <= 0 || c.n_vocab <= 0)
        return (int)hipErrorInvalidValue;
    try {
        std::unique_ptr<tf_model> m(new tf_model());
        m->cfg = c;
        for (int i = 0; i < c.n_layer; i++) {
            const tf_layer& L = layers[i];
            Layer l;
            l.attn_norm = L.attn_norm;
            l.ffn_norm = L.ffn_norm;
            l.wq = to_mat(L.wq);
            l.wk = to_mat(L.wk);
            l.wv = to_mat(L.wv);
            l.wo = to_mat(L.wo);
            l.gate = to_mat(L.gate);
            l.up = to_mat(L.up);
            l.down = to_mat(L.down);
            l.bq = L.bq;
            l.bk = L.bk;
            l.bv = L.bv;
            m->layers.push_back(l);
        }
        m->token_embd = to_mat(*token_embd);
        m->embd_block_bytes = token_embd->type == TF_TYPE_Q6_K   ? 210
                              : token_embd->type == TF_TYPE_Q8_0 ? 34
                              : token_embd->type == TF_TYPE_Q5_0 ? 22
                                                                 : 144;
        m->output = to_mat(*output);
        m->output_norm = output_norm;
        const int n_split = tf_flash_decode_n_split(c.n_kv, c.max_seq);
        m->fd = {c.n_head, c.n_kv, c.head_dim, n_split, 1.0f / std::sqrt((float)c.head_dim)};
        const size_t widest = std::max<size_t>(std::max(c.n_ff, c.n_embd), c.n_vocab);
        m->x = m->alloc<float>(c.n_embd);
        m->xb = m->alloc<float>(c.n_embd);
        m->q = m->alloc<float>(c.n_embd);
        m->k = m->alloc<float>(c.n_kv * c.head_dim);
        m->v = m->alloc<float>(c.n_kv * c.head_dim);
        m->hb = m->alloc<float>(c.n_ff);
        m->hb2 = m->alloc<float>(c.n_ff);
        m->logits = m->alloc<float>(c.n_vocab);
        m->q8_x = m->alloc<int8_t>(std::max(c.n_ff, c.n_embd));
        m->q8_d = m->alloc<float>(std::max(c.n_ff, c.n_embd) / 32);
        m->partial_stride = widest;
        m->gemv_partial = m->alloc<float>(8 * widest);
        m->flash_partial = m->alloc<float>((size_t)c.n_head * n_split * (2 + c.head_dim));
        const size_t kv_elems = (size_t)c.max_seq * c.n_kv * c.head_dim;
        for (int i = 0; i < c.n_layer; i++) {
            m->kc.push_back(m->alloc<uint16_t>(kv_elems));
            m->vc.push_back(m->alloc<uint16_t>(kv_elems));
        }
        m->d_pos = m->alloc<int>(1);
        m->d_step = m->alloc<int>(1);
        m->d_token = m->alloc<int>(1);
        m->d_argmax = m->alloc<int>(1);
        m->d_amax_key = m->alloc<unsigned long long>(TF_ARGMAX_SLOTS);
        tf::check((int)hipMemset(m->d_amax_key, 0, TF_ARGMAX_SLOTS * sizeof(unsigned long long)),
                  "memset");
        m->d_flash_cnt = m->alloc<unsigned>(c.n_kv);
        tf::check((int)hipMemset(m->d_flash_cnt, 0, c.n_kv * sizeof(unsigned)), "memset");
        m->d_nforced = m->alloc<int>(1);
        m->d_forced = m->alloc<int>(c.max_seq);
        m->d_log = m->alloc<int>(c.max_seq);
        // the persistent step where the kernel serves this model, else the
        // fused multi-launch step
        m->path = m->persistent_ok() ? 4 : (m->kquant_ok() ? 3 : 0);
        *out = m.release();
        return 0;
    } catch (const tf::HipError& e) {
        return e.code;
    } catch (const std::bad_alloc&) {
        return (int)hipErrorOutOfMemory;
    }
}

extern "C" void tf_model_destroy(tf_model* m) { delete m; }

extern "C" int tf_model_forward(tf_model* m, int token, int pos, int* next_token,
                                tf_stream_t stream) {
    if (!m || token < 0 || token >= m->cfg.n_vocab || pos < 0 || pos >= m->cfg.max_seq)
        return (int)hipErrorInvalidValue;
    try {
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        m->run_step(s, token, pos, false);
        if (next_token) {
            tf::check((int)hipMemcpyAsync(next_token, m->d_argmax, sizeof(int),
                                          hipMemcpyDeviceToHost, s), "copy");
            tf::check((int)hipStreamSynchronize(s), "sync");
            m->check_persistent(s);
        }
        return 0;
    } catch (const tf::HipError& e) {
        return e.code;
    }
}

extern "C" int tf_model_generate(tf_model* m, const int* forced, int n_forced, int pos0,
                                 int n_gen, int* tokens, int use_graph, tf_stream_t stream) {
    if (!m || !forced || n_forced < 1 || n_gen < 0) return (int)hipErrorInvalidValue;
    for (int i = 0; i < n_forced; i++)
        if (forced[i] < 0 || forced[i] >= m->cfg.n_vocab) return (int)hipErrorInvalidValue;
    try {
        m->run(reinterpret_cast<hipStream_t>(stream), forced, n_forced, pos0, n_gen, tokens,
               use_graph != 0);
        return 0;
    } catch (const tf::HipError& e) {
        return e.code;
    }
}

extern "C" int tf_model_prefill(tf_model* m, const int* tokens, int n_tok, int pos0,
                                int* next_token, tf_stream_t stream) {
    if (!m || !tokens || n_tok < 1 || pos0 < 0) return (int)hipErrorInvalidValue;
    for (int i = 0; i < n_tok; i++)
        if (tokens[i] < 0 || tokens[i] >= m->cfg.n_vocab) return (int)hipErrorInvalidValue;
    try {
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        m->prefill(s, tokens, n_tok, pos0);
        if (next_token)
            tf::check((int)hipMemcpyAsync(next_token, m->d_argmax, sizeof(int),
                                          hipMemcpyDeviceToHost, s), "copy");
        tf::check((int)hipStreamSynchronize(s), "sync");
        return 0;
    } catch (const tf::HipError& e) {
        return e.code;
    } catch (const std::bad_alloc&) {
        return (int)hipErrorOutOfMemory;
    }
}

extern "C" int tf_model_get_path(const tf_model* m) { return m ? m->path : -1; }

extern "C" int tf_model_set_path(tf_model* m, int path) {
    if (!m || path < 0 || path > 4) return (int)hipErrorInvalidValue;
    if (path == 4 && !m->persistent_ok()) return (int)hipErrorNotSupported;
    if (path >= 1 && !m->kquant_ok()) return (int)hipErrorNotSupported;
    if (m->path != path) {
        m->path = path;
        m->drop_graph();
    }
    return 0;
}

extern "C" int tf_model_keep_stage_vectors(tf_model* m, int on) {
    if (!m) return (int)hipErrorInvalidValue;
    if (m->d_players && m->p_keep != (on != 0)) return (int)hipErrorNotSupported;
    if (on && m->cfg.n_layer < 2) return (int)hipErrorInvalidValue;
    m->p_keep = on != 0;
    return 0;
}

extern "C" const unsigned long long* tf_model_stage_vector(const tf_model* m, int kind, int li) {
    if (!m || !m->p_keep || !m->d_players || li < 0 || li >= m->cfg.n_layer) return nullptr;
    const TfPArgs& a = m->pargs;
    switch (kind) {
    case 0: return a.fx + (size_t)li * a.E;                 // residual after wo, f32
    case 1: return a.fx + (size_t)(a.nbuf + li) * a.E;      // residual after down, f32
    case 2: return a.fq + (size_t)li * a.H * a.HD;          // roped query, f32
    case 4: return a.fo + (size_t)li * a.H * a.HD;          // attention output, Q8 groups
    case 5: return a.fh + (size_t)li * a.F;                 // silu(gate)*up, Q8 groups
    default: return nullptr;
    }
}

extern "C" const void* tf_model_q8_record(const tf_model* m, int site, int li, int part) {
    if (!m || !m->p_keep || !m->p_q8x || site < 0 || site > 3 || li < 0 ||
        li > m->cfg.n_layer || part < 0 || part > 2)
        return nullptr;
    const size_t off = ((size_t)li * 4 + (size_t)site) * (size_t)m->p_q8n;
    if (part == 0) return m->p_q8x + off;
    if (part == 1) return m->p_q8q + off;
    return m->p_q8d + off / 32;
}

extern "C" const float* tf_model_logits(const tf_model* m) { return m ? m->logits : nullptr; }
extern "C" uint16_t* tf_model_k_cache(const tf_model* m, int li) {
    return (m && li >= 0 && li < (int)m->kc.size()) ? m->kc[li] : nullptr;
}
extern "C" uint16_t* tf_model_v_cache(const tf_model* m, int li) {
    return (m && li >= 0 && li < (int)m->vc.size()) ? m->vc[li] : nullptr;
}
