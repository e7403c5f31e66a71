// Fused decode-step kernels for gfx950.  Each fuses a chain of reference
// kernels that run back to back on one stream in the reference's decode step
// (cuda/layer.rs) into one launch, so that the step needs six launches per
// layer instead of seventeen:
//   tf_fused_norm_qkv_rope_kv  rms_norm_f32 + quantize_q8 + gemv_q4_k_pair
//                              (Q, K, bias) + gemv_q6_k (V, bias) + 2x
//                              rope_neox_f32 + 2x copy_kv_f16
//                              (layer.rs:171-645)
//   tf_gemv_q4k_ffn_norm       rms_norm_f32 + gemv_q4_k_ffn_mcol
//                              (layer.rs:1220-1386)
//   tf_gemv_q6k_compact_f32    quantize_q8 + gemv_q6_k_compact_global_8way
//                              (down on Q6_K layers, matmul.rs:191-223)
//   tf_gemv_q6k_head_argmax    rms_norm_f32 + quantize_q8 +
//                              gemv_q6_k_compact_global + argmax_f32
//                              (layer.rs:2158-2257)
// Every stage keeps the reference arithmetic of its unfused counterpart: the
// normalization and Q8 bytes are bit-identical, GEMV sums differ only in
// fp32 summation order.
#include <math.h>

#include <type_traits>

#include "q4k.hpp"
#include "q6k.hpp"
#include "argmax_key.hpp"
#include "tf_host.hpp"

struct TfQkvArgs {
    const uint8_t* wq;
    const uint8_t* wk;
    const uint8_t* wv;
    const float* bq;
    const float* bk;
    const float* bv;
    int n_q, n_k, n_v;
    int col_bytes_qk, col_bytes_v, v_q6k;
    float* q_out;
    uint16_t* k_cache;
    uint16_t* v_cache;
    int stride;  // n_kv * head_dim
    int pos;
    const int* pos_dev;
    float theta;
    int head_dim;
};

__device__ __forceinline__ void tf_rope_pair(float x0, float x1, int i, int head_dim, int pos,
                                             float theta, float& y0, float& y1) {
    const float freq = powf(theta, -2.f * (float)i / (float)head_dim);
    const float ang = (float)pos * freq;
    float s, c;
    sincosf(ang, &s, &c);
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}

template <int SPR, int ITERS>
__device__ __forceinline__ float tf_q4k_row(const uint8_t* col, bool valid, int nb, int sir,
                                            int t, const TfAct& x) {
    float acc;
    if constexpr (ITERS > 0) {
        TfQ4kRow<ITERS> r;
        tf_q4k_row_load<SPR, ITERS>(col, valid, 0, nb, sir, t, r);
        acc = tf_q4k_row_partial<SPR, ITERS>(r, valid, 0, nb, sir, t, x);
    } else {
        acc = tf_q4k_row_partial_loop<SPR>(col, valid, 0, nb, sir, t, x);
    }
    return tf_group_sum<4 * SPR>(acc);
}

// Q/K rows are processed as RoPE pairs (i, i + head_dim/2) of one head so the
// rotation happens in registers; V rows follow.  Task map: pair tasks first
// (UNITS/2 pairs per wave pass, or one pair in two passes when a row takes
// the whole wave), then V tasks (UNITS rows per pass).
template <int SPR, int ITERS, int SK>
__global__ __launch_bounds__(TF_BT_QKV) void tf_fused_qkv_kernel(TfQkvArgs a, TfActSrc src, int nb) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int UNITS = 16 / SPR;
    constexpr int PPT = UNITS >= 2 ? UNITS / 2 : 1;
    const int lane = threadIdx.x & 63;
    const int t = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
    const int wave = tf_wave_id();
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    const int hd = a.head_dim, half = hd / 2;
    const int n_pairs = (a.n_q + a.n_k) / 2;
    const int pair_tasks = (n_pairs + PPT - 1) / PPT;
    const int v_tasks = (a.n_v + UNITS - 1) / UNITS;
    const int n_tasks = pair_tasks + v_tasks;
    const int pos = a.pos_dev ? a.pos_dev[0] : a.pos;
    tf_stage_act<true, SK>(src, nb, lds);
    const TfAct x = tf_act_view(lds, nb);
    const bool lead = (lane & (4 * SPR - 1)) == 0;
    for (int task = wave; task < n_tasks; task += nwaves) {
        if (task < pair_tasks) {
            if constexpr (UNITS >= 2) {
                const int pair = task * PPT + unit / 2, member = unit & 1;
                const bool valid = pair < n_pairs;
                const int head = valid ? pair / half : 0, i = valid ? pair % half : 0;
                const int row = head * hd + i + member * half;
                const bool is_q = row < a.n_q;
                const uint8_t* col = is_q ? a.wq + (size_t)row * a.col_bytes_qk
                                          : a.wk + (size_t)(row - a.n_q) * a.col_bytes_qk;
                float acc = tf_q4k_row<SPR, ITERS>(col, valid, nb, sir, t, x);
                if (valid && (is_q ? a.bq : a.bk)) acc += is_q ? a.bq[row] : a.bk[row - a.n_q];
                const float other = __shfl(acc, lane ^ (4 * SPR), 64);
                const float x0 = member == 0 ? acc : other;
                const float x1 = member == 0 ? other : acc;
                float y0, y1;
                tf_rope_pair(x0, x1, i, hd, pos, a.theta, y0, y1);
                const float y = member == 0 ? y0 : y1;
                if (valid && lead) {
                    if (is_q) a.q_out[row] = y;
                    else a.k_cache[(size_t)pos * a.stride + (row - a.n_q)] = tf_f2h_halfup(y);
                }
            } else {
                const int pair = task, head = pair / half, i = pair % half;
                const int r0 = head * hd + i, r1 = r0 + half;
                const bool is_q = r0 < a.n_q;
                const uint8_t* base = is_q ? a.wq : a.wk;
                const int off = is_q ? 0 : a.n_q;
                float x0 = tf_q4k_row<SPR, ITERS>(base + (size_t)(r0 - off) * a.col_bytes_qk, true,
                                                  nb, sir, t, x);
                float x1 = tf_q4k_row<SPR, ITERS>(base + (size_t)(r1 - off) * a.col_bytes_qk, true,
                                                  nb, sir, t, x);
                const float* b = is_q ? a.bq : a.bk;
                if (b) {
                    x0 += b[r0 - off];
                    x1 += b[r1 - off];
                }
                float y0, y1;
                tf_rope_pair(x0, x1, i, hd, pos, a.theta, y0, y1);
                if (lane == 0) {
                    if (is_q) {
                        a.q_out[r0] = y0;
                        a.q_out[r1] = y1;
                    } else {
                        a.k_cache[(size_t)pos * a.stride + (r0 - off)] = tf_f2h_halfup(y0);
                        a.k_cache[(size_t)pos * a.stride + (r1 - off)] = tf_f2h_halfup(y1);
                    }
                }
            }
        } else {
            const int j = (task - pair_tasks) * UNITS + unit;
            const bool valid = j < a.n_v;
            float acc = 0.f;
            if (a.v_q6k) {
                const uint8_t* col = a.wv + (size_t)(valid ? j : 0) * a.col_bytes_v;
                for (int sb = sir; valid && sb < nb; sb += SPR) {
                    TfQ6kPart q;
                    tf_q6k_load_r(col + (size_t)sb * 210, t, q);
                    acc += tf_q6k_f32_part_dot(q, t, sb, x);
                }
                acc = tf_group_sum<4 * SPR>(acc);
            } else {
                acc = tf_q4k_row<SPR, ITERS>(a.wv + (size_t)(valid ? j : 0) * a.col_bytes_v, valid,
                                             nb, sir, t, x);
            }
            if (valid && lead) {
                if (a.bv) acc += a.bv[j];
                a.v_cache[(size_t)pos * a.stride + j] = tf_f2h_halfup(acc);
            }
        }
    }
}

// Q6_K compact rows with an activation source, a residual epilogue and an
// optional argmax (ARGMAX: keys are max-merged per wave, then into the
// wave's slot with one atomicMax).
template <int SPR, int ITERS, bool ARGMAX, int SK>
__global__ __launch_bounds__(tf_bt_rows(SPR)) void tf_q6k_rows_src_kernel(
    const uint8_t* __restrict__ w, TfActSrc src, float* __restrict__ out, int nb, int n_cols,
    int col_bytes, int use_res, unsigned long long* __restrict__ amax) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int UNITS = 16 / SPR;
    const int lane = threadIdx.x & 63;
    const int p = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
    const int wave = tf_wave_id();
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    const int n_tasks = (n_cols + UNITS - 1) / UNITS;
    int task = wave;
    int j = task * UNITS + unit;
    TfQ6kRow<ITERS> cur, nxt;
    if (ITERS > 0 && task < n_tasks)
        tf_q6k_row_load<SPR, ITERS>(w + (size_t)(j < n_cols ? j : 0) * col_bytes, j < n_cols, 0,
                                    nb, sir, p, cur);
    tf_stage_act<false, SK>(src, nb, lds);
    const TfAct x = tf_act_view(lds, nb);
    unsigned long long best = 0;
    for (; task < n_tasks; task += nwaves) {
        const int nt = task + nwaves;
        const int jn = nt * UNITS + unit;
        const bool valid = j < n_cols;
        float acc;
        if constexpr (ITERS > 0) {
            if (nt < n_tasks)
                tf_q6k_row_load<SPR, ITERS>(w + (size_t)(jn < n_cols ? jn : 0) * col_bytes,
                                            jn < n_cols, 0, nb, sir, p, nxt);
            acc = tf_q6k_row_partial<SPR, ITERS>(cur, valid, 0, nb, sir, p, x);
        } else {
            acc = tf_q6k_row_partial_loop<SPR>(w + (size_t)(valid ? j : 0) * col_bytes, valid, 0,
                                               nb, sir, p, x);
        }
        acc = tf_group_sum<4 * SPR>(acc);
        if (valid && (lane & (4 * SPR - 1)) == 0) {
            if (use_res == 2) acc += out[j];
            out[j] = acc;
            if (ARGMAX) {
                const unsigned long long k = tf_argmax_key(acc, j);
                best = k > best ? k : best;
            }
        }
        if constexpr (ITERS > 0) cur = nxt;
        j = jn;
    }
    if (ARGMAX) {
        best = tf_wave_max_u64(best);
        if (lane == 0 && best) atomicMax(amax + (wave % TF_ARGMAX_SLOTS), best);
    }
}

__global__ __launch_bounds__(256) void tf_argmax_key_finalize_kernel(unsigned long long* slots,
                                                                     int* out_idx) {
    const unsigned long long k = tf_argmax_slots_take(slots);
    if (threadIdx.x == 0) *out_idx = tf_argmax_key_index(k);
}

// ---------------------------------------------------------------- dispatch

template <int V>
using tf_icf = std::integral_constant<int, V>;

template <typename F>
static void tf_fused_dispatch(int len, F&& f) {
    if (len <= 4) return f(tf_icf<4>{}, tf_icf<1>{});
    if (len <= 8) return f(tf_icf<8>{}, tf_icf<1>{});
    switch ((len + 15) / 16) {
    case 1: return f(tf_icf<16>{}, tf_icf<1>{});
    case 2: return f(tf_icf<16>{}, tf_icf<2>{});
    case 3: return f(tf_icf<16>{}, tf_icf<3>{});
    case 4: return f(tf_icf<16>{}, tf_icf<4>{});
    case 5: return f(tf_icf<16>{}, tf_icf<5>{});
    default: return f(tf_icf<16>{}, tf_icf<0>{});
    }
}

static TfActSrc tf_src_of(const float* x, const float* norm_w, float eps, int n_x) {
    return TfActSrc{norm_w ? TF_SRC_NORM : TF_SRC_F32, nullptr, nullptr, x, norm_w, eps, n_x};
}

static int tf_q6k_src_launch(const uint8_t* w, const TfActSrc& src, float* out, int n_rows,
                             int n_cols, int col_bytes, int use_res, unsigned long long* amax,
                             tf_stream_t stream) {
    TF_CHECK_ARG(tf_src_ok(src) && src.kind != TF_SRC_FLASH);
    const int nb = n_rows / 256;
    const int lds = tf_act_lds_bytes(nb, false);
    int rc = 0;
    tf_fused_dispatch(nb, [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        const int tasks = (n_cols + 16 / SPR - 1) / (16 / SPR);
        if (amax) {
            auto fn = tf_sk_pick(src.kind, tf_q6k_rows_src_kernel<SPR, IT, true, TF_SRC_Q8>,
                                 tf_q6k_rows_src_kernel<SPR, IT, true, TF_SRC_F32>,
                                 tf_q6k_rows_src_kernel<SPR, IT, true, TF_SRC_NORM>);
            const int BT = tf_block_threads(tf_bt_rows(SPR), tasks);
            const int blocks = tf_persistent_blocks((const void*)fn, BT, lds, tasks);
            hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), lds, tf_stream(stream), w, src, out, nb,
                               n_cols, col_bytes, use_res, amax);
        } else {
            auto fn = tf_sk_pick(src.kind, tf_q6k_rows_src_kernel<SPR, IT, false, TF_SRC_Q8>,
                                 tf_q6k_rows_src_kernel<SPR, IT, false, TF_SRC_F32>,
                                 tf_q6k_rows_src_kernel<SPR, IT, false, TF_SRC_NORM>);
            const int BT = tf_block_threads(tf_bt_rows(SPR), tasks);
            const int blocks = tf_persistent_blocks((const void*)fn, BT, lds, tasks);
            hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), lds, tf_stream(stream), w, src, out, nb,
                               n_cols, col_bytes, use_res, amax);
        }
        rc = TF_LAUNCH_RESULT();
    });
    return rc;
}

// ---------------------------------------------------------------- C ABI

extern "C" int tf_fused_norm_qkv_rope_kv(
    const float* x, const float* norm_w, float eps, const uint8_t* wq, const uint8_t* wk,
    const uint8_t* wv, int v_type, const float* bq, const float* bk, const float* bv, int n_embd,
    int n_head, int n_kv, int head_dim, int col_bytes_qk, int col_bytes_v, float* q_out,
    uint16_t* k_cache, uint16_t* v_cache, int pos, const int* pos_dev, float theta,
    tf_stream_t stream) {
    const int nb = n_embd / 256;
    TF_CHECK_ARG(x && wq && wk && wv && q_out && k_cache && v_cache && nb > 0);
    TF_CHECK_ARG(n_head > 0 && n_kv > 0 && head_dim > 0 && (head_dim & 1) == 0);
    TF_CHECK_ARG(v_type == TF_TYPE_Q4_K || v_type == TF_TYPE_Q6_K);
    TF_CHECK_ARG(((uintptr_t)wq & 15) == 0 && ((uintptr_t)wk & 15) == 0 && (col_bytes_qk & 15) == 0);
    TF_CHECK_ARG(col_bytes_qk >= nb * 144);
    if (v_type == TF_TYPE_Q6_K)
        TF_CHECK_ARG(((uintptr_t)wv & 1) == 0 && (col_bytes_v & 1) == 0 && col_bytes_v >= nb * 210);
    else
        TF_CHECK_ARG(((uintptr_t)wv & 15) == 0 && (col_bytes_v & 15) == 0 && col_bytes_v >= nb * 144);
    TF_CHECK_ARG(pos_dev || pos >= 0);
    TfQkvArgs a{wq, wk, wv, bq, bk, bv, n_head * head_dim, n_kv * head_dim, n_kv * head_dim,
                col_bytes_qk, col_bytes_v, v_type == TF_TYPE_Q6_K ? 1 : 0, q_out, k_cache, v_cache,
                n_kv * head_dim, pos, pos_dev, theta, head_dim};
    const TfActSrc src = tf_src_of(x, norm_w, eps, n_embd);
    TF_CHECK_ARG(tf_src_ok(src) && src.kind != TF_SRC_FLASH);
    const int lds = tf_act_lds_bytes(nb, true);
    int rc = 0;
    tf_fused_dispatch(nb, [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        constexpr int UNITS = 16 / SPR;
        constexpr int PPT = UNITS >= 2 ? UNITS / 2 : 1;
        auto fn = tf_sk_pick(src.kind, tf_fused_qkv_kernel<SPR, IT, TF_SRC_Q8>,
                             tf_fused_qkv_kernel<SPR, IT, TF_SRC_F32>,
                             tf_fused_qkv_kernel<SPR, IT, TF_SRC_NORM>);
        const int tasks = ((a.n_q + a.n_k) / 2 + PPT - 1) / PPT + (a.n_v + UNITS - 1) / UNITS;
        const int BT = tf_block_threads(TF_BT_QKV, tasks);
        const int blocks = tf_persistent_blocks((const void*)fn, BT, lds, tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), lds, tf_stream(stream), a, src, nb);
        rc = TF_LAUNCH_RESULT();
    });
    return rc;
}

extern "C" int tf_fused_qkv_rope_kv(const int8_t* xq, const float* xd, const float* xb,
                                    const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                                    int v_type, const float* bq, const float* bk, const float* bv,
                                    int n_embd, int n_head, int n_kv, int head_dim,
                                    int col_bytes_qk, int col_bytes_v, float* q_out,
                                    uint16_t* k_cache, uint16_t* v_cache, int pos,
                                    const int* pos_dev, float theta, tf_stream_t stream) {
    const int nb = n_embd / 256;
    TF_CHECK_ARG(xq && xd && wq && wk && wv && q_out && k_cache && v_cache && nb > 0);
    TF_CHECK_ARG(n_head > 0 && n_kv > 0 && head_dim > 0 && (head_dim & 1) == 0);
    TF_CHECK_ARG(v_type == TF_TYPE_Q4_K || (v_type == TF_TYPE_Q6_K && xb &&
                                             ((uintptr_t)xb & 15) == 0));
    TF_CHECK_ARG(((uintptr_t)wq & 15) == 0 && ((uintptr_t)wk & 15) == 0 && (col_bytes_qk & 15) == 0);
    TF_CHECK_ARG(col_bytes_qk >= nb * 144);
    if (v_type == TF_TYPE_Q6_K)
        TF_CHECK_ARG(((uintptr_t)wv & 1) == 0 && (col_bytes_v & 1) == 0 && col_bytes_v >= nb * 210);
    else
        TF_CHECK_ARG(((uintptr_t)wv & 15) == 0 && (col_bytes_v & 15) == 0 && col_bytes_v >= nb * 144);
    TF_CHECK_ARG(pos_dev || pos >= 0);
    TfQkvArgs a{wq, wk, wv, bq, bk, bv, n_head * head_dim, n_kv * head_dim, n_kv * head_dim,
                col_bytes_qk, col_bytes_v, v_type == TF_TYPE_Q6_K ? 1 : 0, q_out, k_cache, v_cache,
                n_kv * head_dim, pos, pos_dev, theta, head_dim};
    const TfActSrc src{TF_SRC_Q8, xq, xd, v_type == TF_TYPE_Q6_K ? xb : nullptr, nullptr, 0.f};
    const int lds = tf_act_lds_bytes(nb, true);
    int rc = 0;
    tf_fused_dispatch(nb, [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        constexpr int UNITS = 16 / SPR;
        constexpr int PPT = UNITS >= 2 ? UNITS / 2 : 1;
        auto fn = tf_sk_pick(src.kind, tf_fused_qkv_kernel<SPR, IT, TF_SRC_Q8>,
                             tf_fused_qkv_kernel<SPR, IT, TF_SRC_F32>,
                             tf_fused_qkv_kernel<SPR, IT, TF_SRC_NORM>);
        const int tasks = ((a.n_q + a.n_k) / 2 + PPT - 1) / PPT + (a.n_v + UNITS - 1) / UNITS;
        const int BT = tf_block_threads(TF_BT_QKV, tasks);
        const int blocks = tf_persistent_blocks((const void*)fn, BT, lds, tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), lds, tf_stream(stream), a, src, nb);
        rc = TF_LAUNCH_RESULT();
    });
    return rc;
}

extern "C" int tf_gemv_q6k_q8_argmax(const uint8_t* w, const int8_t* xq, const float* xd,
                                     float* logits, int n_rows, int n_cols, int col_bytes,
                                     unsigned long long* amax_key, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(w && xq && xd && logits && amax_key && nb > 0 && n_cols > 0);
    TF_CHECK_ARG(((uintptr_t)w & 3) == 0 && (col_bytes & 3) == 0 && col_bytes >= nb * 212);
    return tf_q6k_src_launch(w, TfActSrc{TF_SRC_Q8, xq, xd, nullptr, nullptr, 0.f}, logits,
                             n_rows, n_cols, col_bytes, 0, amax_key, stream);
}

extern "C" int tf_gemv_q6k_compact_f32(const uint8_t* w, const float* x, float* out, int n_rows,
                                       int n_cols, int col_bytes, int use_res,
                                       tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(w && x && out && nb > 0 && n_cols > 0 && (use_res == 0 || use_res == 2));
    TF_CHECK_ARG(((uintptr_t)w & 3) == 0 && (col_bytes & 3) == 0 && col_bytes >= nb * 212);
    return tf_q6k_src_launch(w, tf_src_of(x, nullptr, 0.f, n_rows), out, n_rows, n_cols, col_bytes,
                             use_res, nullptr, stream);
}

extern "C" int tf_gemv_q6k_head_argmax(const uint8_t* w, const float* x, const float* norm_w,
                                       float eps, float* logits, int n_rows, int n_cols,
                                       int col_bytes, unsigned long long* amax_key,
                                       tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(w && x && logits && amax_key && nb > 0 && n_cols > 0);
    TF_CHECK_ARG(((uintptr_t)w & 3) == 0 && (col_bytes & 3) == 0 && col_bytes >= nb * 212);
    return tf_q6k_src_launch(w, tf_src_of(x, norm_w, eps, n_rows), logits, n_rows, n_cols, col_bytes, 0,
                             amax_key, stream);
}

extern "C" int tf_argmax_key_finalize(unsigned long long* amax_key, int* out_idx,
                                      tf_stream_t stream) {
    TF_CHECK_ARG(amax_key && out_idx);
    hipLaunchKernelGGL(tf_argmax_key_finalize_kernel, dim3(1), dim3(256), 0, tf_stream(stream),
                       amax_key, out_idx);
    return TF_LAUNCH_RESULT();
}
