// C++ operator API of the decode path: the host-side interface the reference
// exposes to its model runtime in cuda/matmul.rs and the flash branch of
// cuda/layer.rs:2040-2121, restated over this library's C ABI.
//
// Names, argument meaning and the bool "not applicable" protocol of the
// try_* functions follow matmul.rs; errors are raised as tf::HipError (the
// reference returns anyhow::Error).  Kernel selection is MI355X-specific:
// where the reference splits a tall GEMV into split-K partials plus a reduce
// (matmul.rs:225-283) the full-K single-pass kernel is used, because one
// wave already owns a whole row and the partial round trip only adds a
// launch; results agree within the fp32 GEMV tolerance.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "taraference_hip.h"

namespace tf {

enum class WType { Q4K, Q6K, Q5_0, Q8_0 };

// cuda/types.rs:212-225
struct GpuMat {
    const uint8_t* data = nullptr;
    const uint8_t* compact_data = nullptr;  // 212-byte Q6_K repack
    size_t n_rows = 0;                       // K (input length)
    size_t n_cols = 0;                       // N (outputs)
    size_t col_bytes = 0;
    size_t compact_col_bytes = 0;
    WType wtype = WType::Q4K;
};

// matmul.rs:106-114
struct GemvResidual {
    enum Kind { None, Add, InPlace } kind = None;
    const float* add = nullptr;
    static GemvResidual none() { return {}; }
    static GemvResidual in_place() { return {InPlace, nullptr}; }
    static GemvResidual add_from(const float* r) { return {Add, r}; }
    int use_res() const { return kind == None ? 0 : (kind == Add ? 1 : 2); }
};

struct HipError : std::runtime_error {
    int code;
    HipError(int c, const std::string& what) : std::runtime_error(what), code(c) {}
};

void check(int rc, const char* what);

// matmul.rs:47 quantize_q8
void quantize_q8(hipStream_t s, const float* x, int8_t* q8_x, float* q8_d, int n_rows);

// matmul.rs:96-104 gemv_n_split (dispatch policy of the reference; reported
// for parity of selection, see the file comment for how it is used)
uint32_t gemv_n_split(size_t n_rows);

// matmul.rs:118 gemv: y = W x [+bias] [+residual] with an f32 activation.
void gemv(hipStream_t s, const GpuMat& w, const float* x, float* y, const float* bias,
          GemvResidual res, float* partial, size_t partial_stride);

// matmul.rs:142 try_gemv_global_q8: quantize x once, then the Q8 GEMV.
bool try_gemv_global_q8(hipStream_t s, const GpuMat& w, const float* x, float* y,
                        const float* bias, GemvResidual res, int8_t* q8_x, float* q8_d,
                        float* partial, size_t partial_stride);

// matmul.rs:509 try_gemv_pair (Q4_K branch :727-784)
bool try_gemv_pair(hipStream_t s, const GpuMat& wa, const GpuMat& wb, const float* x,
                   float* out_a, float* out_b, const float* ba, const float* bb, int8_t* q8_x,
                   float* q8_d);

// matmul.rs:582 try_gemv_q4_dual
bool try_gemv_q4_dual(hipStream_t s, const GpuMat& wa, const GpuMat& wb, const float* x,
                      float* out_a, float* out_b, int8_t* q8_x, float* q8_d);

// matmul.rs:786 try_gemv_q5_dual (Q+K or gate+up, both Q5_0, f32 x)
bool try_gemv_q5_dual(hipStream_t s, const GpuMat& wa, const GpuMat& wb, const float* x,
                      float* out_a, float* out_b, const float* ba, const float* bb);

// matmul.rs:627 try_gemv_q4_ffn: out = silu(gate x) * (up x)
bool try_gemv_q4_ffn(hipStream_t s, const GpuMat& gate, const GpuMat& up, const float* x,
                     float* out, int8_t* q8_x, float* q8_d);

// matmul.rs:926 try_gemv_qkv (Q4_K branch :962-1002)
bool try_gemv_qkv(hipStream_t s, const GpuMat& wq, const GpuMat& wk, const GpuMat& wv,
                  const float* x, float* q, float* k, float* v, const float* bq,
                  const float* bk, const float* bv, int8_t* q8_x, float* q8_d);

// layer.rs:2040-2121 flash branch of launch_attn_spec (n_tok = 1).
struct FlashDims {
    int n_head, n_kv, head_dim, n_split;
    float scale;
};
void launch_attn_flash(hipStream_t s, const FlashDims& d, const float* q, const uint16_t* k_cache,
                       const uint16_t* v_cache, float* flash_partial, float* out, int pos0,
                       const int* pos0_dev);

}  // namespace tf
