// Operator API over the C ABI (see op_api.hpp).
#include "op_api.hpp"

namespace tf {

namespace {
constexpr size_t kSplitMinRows = 4096;          // matmul.rs:19
constexpr size_t kBaselineSmemCap = 24 * 1024;  // matmul.rs:21
constexpr uint32_t kSplitMax = 8;               // matmul.rs:16

tf_stream_t S(hipStream_t s) { return reinterpret_cast<tf_stream_t>(s); }
int I(size_t v) { return static_cast<int>(v); }
}  // namespace

void check(int rc, const char* what) {
    if (rc != 0) throw HipError(rc, std::string(what) + " failed with hipError " + std::to_string(rc));
}

void quantize_q8(hipStream_t s, const float* x, int8_t* q8_x, float* q8_d, int n_rows) {
    check(tf_quantize_q8(x, q8_x, q8_d, n_rows, S(s)), "quantize_q8");
}

uint32_t gemv_n_split(size_t n_rows) {
    if (n_rows < kSplitMinRows && n_rows * 4 <= kBaselineSmemCap) return 1;
    return 4u < kSplitMax ? 4u : kSplitMax;
}

void gemv(hipStream_t s, const GpuMat& w, const float* x, float* y, const float* bias,
          GemvResidual res, float* /*partial*/, size_t /*partial_stride*/) {
    const int use_bias = bias ? 1 : 0;
    if (w.wtype == WType::Q5_0) {
        check(tf_gemv_q5_0_f32(w.data, x, y, I(w.n_rows), I(w.n_cols), I(w.col_bytes), use_bias,
                               bias, res.use_res(), res.add, S(s)),
              "gemv_q5_0");
    } else if (w.wtype == WType::Q8_0) {  // x quantized per workgroup (gemv_q8_0)
        check(tf_gemv_q8_0_f32(w.data, x, y, I(w.n_rows), I(w.n_cols), I(w.col_bytes), use_bias,
                               bias, res.use_res(), res.add, S(s)),
              "gemv_q8_0");
    } else if (w.wtype == WType::Q6K) {
        check(tf_gemv_q6k_f32(w.data, x, y, I(w.n_rows), I(w.n_cols), I(w.col_bytes), use_bias,
                              bias, res.use_res(), res.add, S(s)),
              "gemv_q6_k");
    } else {
        check(tf_gemv_q4k_f32(w.data, x, y, I(w.n_rows), I(w.n_cols), I(w.col_bytes), use_bias,
                              bias, res.use_res(), res.add, S(s)),
              "gemv_q4_k");
    }
}

bool try_gemv_global_q8(hipStream_t s, const GpuMat& w, const float* x, float* y,
                        const float* bias, GemvResidual res, int8_t* q8_x, float* q8_d,
                        float* /*partial*/, size_t /*partial_stride*/) {
    if (w.wtype == WType::Q6K && !w.compact_data) return false;
    if (w.wtype == WType::Q5_0) return false;  // no global-Q8 Q5_0 kernel (matmul.rs:160-176)
    const int use_bias = bias ? 1 : 0;
    quantize_q8(s, x, q8_x, q8_d, I(w.n_rows));
    if (w.wtype == WType::Q8_0) {
        check(tf_gemv_q8_0_q8(w.data, q8_x, q8_d, y, I(w.n_rows), I(w.n_cols), I(w.col_bytes),
                              use_bias, bias, res.use_res(), res.add, S(s)),
              "gemv_q8_0_global");
        return true;
    }
    if (w.wtype == WType::Q4K) {
        check(tf_gemv_q4k_q8(w.data, q8_x, q8_d, y, I(w.n_rows), I(w.n_cols), I(w.col_bytes),
                             use_bias, bias, res.use_res(), res.add, S(s)),
              "gemv_q4_k_global");
        return true;
    }
    // Q6_K compact: the reference picks the 8/4-way in-block split-K kernel
    // for tall rows (matmul.rs:196-223) and the single-pass kernel otherwise.
    if (gemv_n_split(w.n_rows) >= 4) {
        check(tf_gemv_q6k_down_splitk(w.compact_data, q8_x, q8_d, y, I(w.n_rows), I(w.n_cols),
                                      I(w.compact_col_bytes), use_bias, bias, res.use_res(),
                                      res.add, S(s)),
              "gemv_q6_k_compact_global_8way");
    } else {
        check(tf_gemv_q6k_compact_q8(w.compact_data, q8_x, q8_d, y, I(w.n_rows), I(w.n_cols),
                                     I(w.compact_col_bytes), use_bias, bias, res.use_res(),
                                     res.add, S(s)),
              "gemv_q6_k_compact_global");
    }
    return true;
}

bool try_gemv_pair(hipStream_t s, const GpuMat& wa, const GpuMat& wb, const float* x,
                   float* out_a, float* out_b, const float* ba, const float* bb, int8_t* q8_x,
                   float* q8_d) {
    if (wa.wtype != WType::Q4K || wb.wtype != WType::Q4K || wa.n_rows != wb.n_rows ||
        wa.col_bytes != wb.col_bytes)
        return false;
    const bool both = ba && bb, none = !ba && !bb;
    if (!both && !none) return false;
    quantize_q8(s, x, q8_x, q8_d, I(wa.n_rows));
    check(tf_gemv_q4k_pair(wa.data, wb.data, q8_x, q8_d, out_a, out_b, I(wa.n_rows),
                           I(wa.n_cols), I(wb.n_cols), I(wa.col_bytes), both ? 1 : 0, ba, bb,
                           S(s)),
          "gemv_q4_k_pair");
    return true;
}

bool try_gemv_q4_dual(hipStream_t s, const GpuMat& wa, const GpuMat& wb, const float* x,
                      float* out_a, float* out_b, int8_t* q8_x, float* q8_d) {
    if (wa.wtype != WType::Q4K || wb.wtype != WType::Q4K || wa.n_rows != wb.n_rows ||
        wa.n_cols != wb.n_cols || wa.col_bytes != wb.col_bytes)
        return false;
    quantize_q8(s, x, q8_x, q8_d, I(wa.n_rows));
    check(tf_gemv_q4k_dual(wa.data, wb.data, q8_x, q8_d, out_a, out_b, I(wa.n_rows),
                           I(wa.n_cols), I(wa.col_bytes), S(s)),
          "gemv_q4_k_dual");
    return true;
}

bool try_gemv_q5_dual(hipStream_t s, const GpuMat& wa, const GpuMat& wb, const float* x,
                      float* out_a, float* out_b, const float* ba, const float* bb) {
    if (wa.wtype != WType::Q5_0 || wb.wtype != WType::Q5_0 || wa.n_rows != wb.n_rows ||
        wa.col_bytes != wb.col_bytes)
        return false;
    const bool both = ba && bb, none = !ba && !bb;
    if (!both && !none) return false;
    check(tf_gemv_q5_0_qk(wa.data, wb.data, x, out_a, out_b, I(wa.n_rows), I(wa.n_cols),
                          I(wb.n_cols), I(wa.col_bytes), both ? 1 : 0, ba, bb, S(s)),
          "gemv_q5_0_qk");
    return true;
}

bool try_gemv_q4_ffn(hipStream_t s, const GpuMat& gate, const GpuMat& up, const float* x,
                     float* out, int8_t* q8_x, float* q8_d) {
    if (gate.wtype != WType::Q4K || up.wtype != WType::Q4K || gate.n_rows != up.n_rows ||
        gate.n_cols != up.n_cols || gate.col_bytes != up.col_bytes)
        return false;
    // Quantize once globally, then the fused gate+up+SiLU kernel
    // (matmul.rs:678-725 choose between in-block and global quantization).
    quantize_q8(s, x, q8_x, q8_d, I(gate.n_rows));
    check(tf_gemv_q4k_ffn(gate.data, up.data, q8_x, q8_d, out, I(gate.n_rows), I(gate.n_cols),
                          I(gate.col_bytes), S(s)),
          "gemv_q4_k_ffn");
    return true;
}

bool try_gemv_qkv(hipStream_t s, const GpuMat& wq, const GpuMat& wk, const GpuMat& wv,
                  const float* x, float* q, float* k, float* v, const float* bq,
                  const float* bk, const float* bv, int8_t* q8_x, float* q8_d) {
    const bool same = wq.n_rows == wk.n_rows && wq.n_rows == wv.n_rows &&
                      wq.col_bytes == wk.col_bytes && wq.col_bytes == wv.col_bytes;
    const bool all = bq && bk && bv, none = !bq && !bk && !bv;
    if (!same || !(all || none)) return false;
    // matmul.rs:1003-1130: all three Q8_0 (x quantized in the kernel), or all
    // three Q5_0 (f32 x)
    if (wq.wtype == WType::Q8_0 && wk.wtype == WType::Q8_0 && wv.wtype == WType::Q8_0) {
        check(tf_gemv_q8_0_qkv(wq.data, wk.data, wv.data, x, q, k, v, I(wq.n_rows), I(wq.n_cols),
                               I(wk.n_cols), I(wv.n_cols), I(wq.col_bytes), all ? 1 : 0, bq, bk,
                               bv, S(s)),
              "gemv_q8_0_qkv");
        return true;
    }
    if (wq.wtype == WType::Q5_0 && wk.wtype == WType::Q5_0 && wv.wtype == WType::Q5_0) {
        check(tf_gemv_q5_0_qkv(wq.data, wk.data, wv.data, x, q, k, v, I(wq.n_rows), I(wq.n_cols),
                               I(wk.n_cols), I(wv.n_cols), I(wq.col_bytes), all ? 1 : 0, bq, bk,
                               bv, S(s)),
              "gemv_q5_0_qkv");
        return true;
    }
    if (wq.wtype != WType::Q4K || wk.wtype != WType::Q4K || wv.wtype != WType::Q4K)
        return false;
    quantize_q8(s, x, q8_x, q8_d, I(wq.n_rows));
    check(tf_gemv_q4k_qkv(wq.data, wk.data, wv.data, q8_x, q8_d, q, k, v, I(wq.n_rows),
                          I(wq.n_cols), I(wk.n_cols), I(wv.n_cols), I(wq.col_bytes), all ? 1 : 0,
                          bq, bk, bv, S(s)),
          "gemv_q4_k_qkv");
    return true;
}

void launch_attn_flash(hipStream_t s, const FlashDims& d, const float* q, const uint16_t* k_cache,
                       const uint16_t* v_cache, float* flash_partial, float* out, int pos0,
                       const int* pos0_dev) {
    if (pos0_dev)
        check(tf_flash_decode_partial_d(q, k_cache, v_cache, flash_partial, d.n_head, d.n_kv,
                                        d.head_dim, pos0_dev, 1, d.n_split, d.scale, S(s)),
              "attn_flash_partial_d");
    else
        check(tf_flash_decode_partial(q, k_cache, v_cache, flash_partial, d.n_head, d.n_kv,
                                      d.head_dim, pos0, 1, d.n_split, d.scale, S(s)),
              "attn_flash_partial");
    check(tf_flash_decode_reduce(flash_partial, out, d.n_head, d.head_dim, d.n_split, 1, S(s)),
          "attn_flash_reduce");
}

}  // namespace tf
