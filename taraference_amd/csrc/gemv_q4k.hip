// Q4_K x Q8 GEMV family for gfx950 (batch 1).
//
// Replaces kernels/gemv.cu gemv_q4_k_global (:469), gemv_q4_k_global_splitk
// (:1877), gemv_splitk_reduce (:2243), gemv_q4_k_pair (:2346),
// gemv_q4_k_dual (:2401), gemv_q4_k_ffn{,_4way,_8way} (:2440-2619),
// gemv_q4_k_ffn_mcol (:2546) and gemv_q4_k_qkv (:2662).
//
// Every kernel is a persistent grid of workgroups sized from the occupancy
// of the kernel: each workgroup stages the activation in LDS once, then each
// wave loops over row tasks.  See q4k.hpp for the lane map.
#include <type_traits>

#include "q4k.hpp"
#include "tf_host.hpp"

// ------------------------------------------------------------------ kernels

struct TfQ4kMats {
    const uint8_t* w0;
    const uint8_t* w1;
    const uint8_t* w2;
    float* o0;
    float* o1;
    float* o2;
    const float* b0;
    const float* b1;
    const float* b2;
    int n0, n1, n2;
};

// Row task helpers.  A wave task covers UNITS = 16/SPR rows at once; every
// kernel below keeps the next task's weights in flight (registers) while it
// computes the current one, and issues its first task's loads before the
// workgroup stages the activation in LDS.

struct TfRowSel {
    const uint8_t* col;
    bool valid;
    int j;   // output index within its matrix
    int mi;  // matrix index
};

__device__ __forceinline__ TfRowSel tf_sel3(const TfQ4kMats& m, int r, int n_total,
                                            int col_bytes) {
    TfRowSel s;
    s.valid = r < n_total;
    int j = s.valid ? r : 0, mi = 0;
    if (j >= m.n0) {
        j -= m.n0;
        mi = 1;
        if (j >= m.n1) {
            j -= m.n1;
            mi = 2;
        }
    }
    s.j = j;
    s.mi = mi;
    s.col = (mi == 0 ? m.w0 : (mi == 1 ? m.w1 : m.w2)) + (size_t)j * col_bytes;
    return s;
}

// Rows of up to three matrices that share K (global / pair / qkv).
template <int SPR, int ITERS, int SK>
__global__ __launch_bounds__(tf_bt_rows(SPR, SK)) void tf_q4k_rows_kernel(
    TfQ4kMats m, TfActSrc src, int nb, int col_bytes, int use_bias, int use_res,
    const float* __restrict__ residual) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int UNITS = 16 / SPR;
    const int lane = threadIdx.x & 63;
    const int t = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
    const int wave = tf_wave_id();
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    const int n_total = m.n0 + m.n1 + m.n2;
    const int n_tasks = (n_total + UNITS - 1) / UNITS;
    int task = wave;
    TfRowSel cs = tf_sel3(m, task * UNITS + unit, n_total, col_bytes);
    TfQ4kRow<ITERS> cur, nxt;
    // A wide activation (16 super-blocks or more) is staged before the first
    // weight loads: issued after them, its loads would complete only behind
    // them (in issue order), and the staging would then lengthen the critical
    // path (Q6_K 11008 -> 2048: 7.6 -> 7.1 us back to back); a narrow one costs
    // less than the delay it would add to the weight stream.
    const bool act_first = nb >= 16;
    if (act_first) tf_stage_act<false, SK>(src, nb, lds);
    if (ITERS > 0 && task < n_tasks) tf_q4k_row_load<SPR, ITERS>(cs.col, cs.valid, 0, nb, sir, t, cur);
    if (!act_first) tf_stage_act<false, SK>(src, nb, lds);
    const TfAct x = tf_act_view(lds, nb);
    for (; task < n_tasks; task += nwaves) {
        const int nt = task + nwaves;
        const TfRowSel ns = tf_sel3(m, nt * UNITS + unit, n_total, col_bytes);
        float acc;
        if constexpr (ITERS > 0) {
            if (nt < n_tasks) tf_q4k_row_load<SPR, ITERS>(ns.col, ns.valid, 0, nb, sir, t, nxt);
            acc = tf_q4k_row_partial<SPR, ITERS>(cur, cs.valid, 0, nb, sir, t, x);
        } else {
            acc = tf_q4k_row_partial_loop<SPR>(cs.col, cs.valid, 0, nb, sir, t, x);
        }
        acc = tf_group_sum<4 * SPR>(acc);
        if (cs.valid && (lane & (4 * SPR - 1)) == 0) {
            const int j = cs.j, mi = cs.mi;
            float* out = mi == 0 ? m.o0 : (mi == 1 ? m.o1 : m.o2);
            if (use_res == 1) acc += residual[j];
            else if (use_res == 2) acc += out[j];
            if (use_bias) acc += (mi == 0 ? m.b0 : (mi == 1 ? m.b1 : m.b2))[j];
            out[j] = acc;
        }
        if constexpr (ITERS > 0) cur = nxt;
        cs = ns;
    }
}

// Narrow rows (at most eight super-blocks) with a Q8 activation: the lanes
// read the activation bytes from global memory right behind their weight
// loads instead of staging an LDS image first (no staging round trip, no
// barrier); arithmetic as tf_q4k_rows_kernel.  It pays where a wave has one
// or two tasks (config 0: 3.72 -> 3.25 us, config 1c: 4.05 -> 3.57 us back to
// back); the fused gate+up at 2048 -> 2 x 11008, five or six tasks per wave,
// went 7.23 -> 8.84 us with it (every task re-reads the activation through
// the memory queue its weight prefetch is in), so the pair keeps the image;
// so does the Q6_K down at K = 11008 (one task per wave, but as many
// activation bytes per lane as weight bytes: 7.03 -> 7.67 us).
template <int SPR, int ITERS>
__global__ __launch_bounds__(tf_bt_rows(SPR)) void tf_q4k_rows_gq8_kernel(
    TfQ4kMats m, const int8_t* __restrict__ xq, const float* __restrict__ xd, int nb,
    int col_bytes, int use_bias, int use_res, const float* __restrict__ residual) {
    constexpr int UNITS = 16 / SPR;
    const int lane = threadIdx.x & 63;
    const int t = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
    const int wave = tf_wave_id();
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    const int n_total = m.n0 + m.n1 + m.n2;
    const int n_tasks = (n_total + UNITS - 1) / UNITS;
    int task = wave;
    TfRowSel cs = tf_sel3(m, task * UNITS + unit, n_total, col_bytes);
    TfQ4kRow<ITERS> cur, nxt;
    if (task < n_tasks) tf_q4k_row_load_u<SPR, ITERS>(cs.col, nb, sir, t, cur);
    for (; task < n_tasks; task += nwaves) {
        const int nt = task + nwaves;
        const TfRowSel ns = tf_sel3(m, nt * UNITS + unit, n_total, col_bytes);
        if (nt < n_tasks) tf_q4k_row_load_u<SPR, ITERS>(ns.col, nb, sir, t, nxt);
        float acc = tf_q4k_row_partial_g<SPR, ITERS>(cur, cs.valid, nb, sir, t, xq, xd);
        acc = tf_group_sum<4 * SPR>(acc);
        if (cs.valid && (lane & (4 * SPR - 1)) == 0) {
            const int j = cs.j, mi = cs.mi;
            float* out = mi == 0 ? m.o0 : (mi == 1 ? m.o1 : m.o2);
            if (use_res == 1) acc += residual[j];
            else if (use_res == 2) acc += out[j];
            if (use_bias) acc += (mi == 0 ? m.b0 : (mi == 1 ? m.b1 : m.b2))[j];
            out[j] = acc;
        }
        cur = nxt;
        cs = ns;
    }
}

template <int MODE>
__device__ __forceinline__ void tf_pair_write(float g, float u, float* out_a, float* out_b,
                                              int j) {
    if constexpr (MODE == 0) {
        out_a[j] = (g / (1.f + __expf(-g))) * u;
    } else {
        out_a[j] = g;
        out_b[j] = u;
    }
}

// Equal-width pair on the same output index: MODE 0 writes
// silu(gate)*up (ffn), MODE 1 writes both dots (dual).  xf != nullptr means
// the activation is f32 and is quantized into LDS by each workgroup.
template <int SPR, int ITERS, int MODE, int SK>
__global__ __launch_bounds__(tf_bt_pair(SPR)) void tf_q4k_pair_rows_kernel(
    const uint8_t* __restrict__ wa, const uint8_t* __restrict__ wb,
    TfActSrc src, float* __restrict__ out_a, float* __restrict__ out_b, int nb, int n_cols,
    int col_bytes) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int t = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
    const int wave = tf_wave_id();
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    if constexpr (SPR <= 8) {
        // even unit = gate row j, odd unit = up row j
        constexpr int JPW = 16 / SPR / 2;
        const int n_tasks = (n_cols + JPW - 1) / JPW;
        const uint8_t* w = (unit & 1) ? wb : wa;
        int task = wave;
        int j = task * JPW + (unit >> 1);
        TfQ4kRow<ITERS> cur, nxt;
        if (task < n_tasks)
            tf_q4k_row_load<SPR, ITERS>(w + (size_t)j * col_bytes, j < n_cols, 0, nb, sir, t, cur);
        tf_stage_act<false, SK>(src, nb, lds);
        const TfAct x = tf_act_view(lds, nb);
        for (; task < n_tasks; task += nwaves) {
            const int nt = task + nwaves;
            const int jn = nt * JPW + (unit >> 1);
            if (nt < n_tasks)
                tf_q4k_row_load<SPR, ITERS>(w + (size_t)jn * col_bytes, jn < n_cols, 0, nb, sir,
                                            t, nxt);
            float acc = tf_q4k_row_partial<SPR, ITERS>(cur, j < n_cols, 0, nb, sir, t, x);
            acc = tf_group_sum<4 * SPR>(acc);
            const float other = __shfl(acc, (lane + 4 * SPR) & 63, 64);
            if (j < n_cols && (unit & 1) == 0 && (lane & (4 * SPR - 1)) == 0)
                tf_pair_write<MODE>(acc, other, out_a, out_b, j);
            cur = nxt;
            j = jn;
        }
    } else {
        int j = wave;
        TfQ4kRow<ITERS> cg, cu, ng, nu;
        if (ITERS > 0 && j < n_cols) {
            tf_q4k_row_load<SPR, ITERS>(wa + (size_t)j * col_bytes, true, 0, nb, sir, t, cg);
            tf_q4k_row_load<SPR, ITERS>(wb + (size_t)j * col_bytes, true, 0, nb, sir, t, cu);
        }
        tf_stage_act<false, SK>(src, nb, lds);
        const TfAct x = tf_act_view(lds, nb);
        for (; j < n_cols; j += nwaves) {
            const int jn = j + nwaves;
            float g, u;
            if constexpr (ITERS > 0) {
                if (jn < n_cols) {
                    tf_q4k_row_load<SPR, ITERS>(wa + (size_t)jn * col_bytes, true, 0, nb, sir, t, ng);
                    tf_q4k_row_load<SPR, ITERS>(wb + (size_t)jn * col_bytes, true, 0, nb, sir, t, nu);
                }
                g = tf_q4k_row_partial<SPR, ITERS>(cg, true, 0, nb, sir, t, x);
                u = tf_q4k_row_partial<SPR, ITERS>(cu, true, 0, nb, sir, t, x);
            } else {
                g = tf_q4k_row_partial_loop<SPR>(wa + (size_t)j * col_bytes, true, 0, nb, sir, t, x);
                u = tf_q4k_row_partial_loop<SPR>(wb + (size_t)j * col_bytes, true, 0, nb, sir, t, x);
            }
            g = tf_group_sum<64>(g);
            u = tf_group_sum<64>(u);
            if (lane == 0) tf_pair_write<MODE>(g, u, out_a, out_b, j);
            if constexpr (ITERS > 0) {
                cg = ng;
                cu = nu;
            }
        }
    }
}

// Split-K partials: task (s, j) covers super-blocks
// [floor(nb*s/n_split), floor(nb*(s+1)/n_split)).
template <int SPR, int ITERS>
__global__ __launch_bounds__(256) void tf_q4k_splitk_kernel(
    const uint8_t* __restrict__ w, TfActSrc src, float* __restrict__ partial, int nb,
    int n_cols, int col_bytes, int n_split) {
    extern __shared__ __align__(16) uint8_t lds[];
    tf_stage_act<false, TF_SRC_Q8>(src, nb, lds);
    const TfAct x = tf_act_view(lds, nb);
    constexpr int UNITS = 16 / SPR;
    const int lane = threadIdx.x & 63;
    const int t = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
    const int wave = tf_wave_id();
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    const int n_total = n_split * n_cols;
    for (int r0 = wave * UNITS; r0 < n_total; r0 += nwaves * UNITS) {
        const int r = r0 + unit;
        const bool valid = r < n_total;
        const int s = valid ? r / n_cols : 0;
        const int j = valid ? r - s * n_cols : 0;
        const int sb0 = (nb * s) / n_split, sb1 = (nb * (s + 1)) / n_split;
        const uint8_t* col = w + (size_t)j * col_bytes;
        float acc;
        if constexpr (ITERS > 0) {
            TfQ4kRow<ITERS> rr;
            tf_q4k_row_load<SPR, ITERS>(col, valid, sb0, sb1, sir, t, rr);
            acc = tf_q4k_row_partial<SPR, ITERS>(rr, valid, sb0, sb1, sir, t, x);
        } else {
            acc = tf_q4k_row_partial_loop<SPR>(col, valid, sb0, sb1, sir, t, x);
        }
        acc = tf_group_sum<4 * SPR>(acc);
        if (valid && (lane & (4 * SPR - 1)) == 0) partial[(size_t)s * n_cols + j] = acc;
    }
}

__global__ __launch_bounds__(256) void tf_splitk_reduce_kernel(
    const float* __restrict__ partial, float* __restrict__ out, int n_cols,
    int n_split, int use_bias, const float* __restrict__ bias, int use_res,
    const float* __restrict__ residual) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n_cols) return;
    float acc = 0.f;
    for (int s = 0; s < n_split; s++) acc += partial[(size_t)s * n_cols + j];
    if (use_res == 1) acc += residual[j];
    else if (use_res == 2) acc += out[j];
    if (use_bias) acc += bias[j];
    out[j] = acc;
}

// Integer diagnostics: the exact stage of tf_q4k_part_dot.
__global__ __launch_bounds__(256) void tf_q4k_block_dots_kernel(
    const uint8_t* __restrict__ w, const int8_t* __restrict__ xq,
    int32_t* __restrict__ dots, int32_t* __restrict__ sums, int nb, int n_cols,
    int col_bytes) {
    extern __shared__ __align__(16) uint8_t lds[];
    int32_t* lsums = reinterpret_cast<int32_t*>(lds + TF_Q8_LDS_BYTES(nb));
    // Same copy-and-sum as tf_stage_act(TF_SRC_Q8); only the integer sums are kept.
    {
        int8_t* q8s = reinterpret_cast<int8_t*>(lds);
        for (int g = threadIdx.x; g < nb * 8; g += blockDim.x) {
            tf_u32x4 a = tf_ld16(xq + g * 32), b = tf_ld16(xq + g * 32 + 16);
            reinterpret_cast<tf_u32x4*>(q8s + tf_q8_pad(g * 32))[0] = a;
            reinterpret_cast<tf_u32x4*>(q8s + tf_q8_pad(g * 32))[1] = b;
            const int one = 0x01010101;
            int s = tf_dot4(one, (int)a.x, 0);
            s = tf_dot4(one, (int)a.y, s);
            s = tf_dot4(one, (int)a.z, s);
            s = tf_dot4(one, (int)a.w, s);
            s = tf_dot4(one, (int)b.x, s);
            s = tf_dot4(one, (int)b.y, s);
            s = tf_dot4(one, (int)b.z, s);
            s = tf_dot4(one, (int)b.w, s);
            lsums[g] = s;
        }
        __syncthreads();
    }
    const int8_t* q8s = reinterpret_cast<const int8_t*>(lds);
    const long long task = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)n_cols * nb * 4;
    if (task >= total) return;
    const int t = (int)(task & 3);
    const long long blk = task >> 2;
    const int j = (int)(blk / nb), sb = (int)(blk % nb);
    TfQ4kPart p;
    tf_q4k_load(w + (size_t)j * col_bytes + (size_t)sb * 144, t, p);
    int dlo, dhi;
    tf_q4k_idots(p, q8s + tf_q8_pad(sb * 256 + 64 * t), dlo, dhi);
    const size_t o = ((size_t)j * nb + sb) * 8 + 2 * t;
    dots[o] = dlo;
    dots[o + 1] = dhi;
    sums[o] = lsums[sb * 8 + 2 * t];
    sums[o + 1] = lsums[sb * 8 + 2 * t + 1];
}

// ---------------------------------------------------------------- dispatch

template <int V>
using tf_ic = std::integral_constant<int, V>;

// Pick slots-per-row and unroll depth for rows of `len` super-blocks.
template <typename F>
static void tf_q4k_dispatch(int len, F&& f) {
    if (len <= 4) return f(tf_ic<4>{}, tf_ic<1>{});
    if (len <= 8) return f(tf_ic<8>{}, tf_ic<1>{});
    switch ((len + 15) / 16) {
    case 1: return f(tf_ic<16>{}, tf_ic<1>{});
    case 2: return f(tf_ic<16>{}, tf_ic<2>{});
    case 3: return f(tf_ic<16>{}, tf_ic<3>{});
    case 4: return f(tf_ic<16>{}, tf_ic<4>{});
    case 5: return f(tf_ic<16>{}, tf_ic<5>{});
    default: return f(tf_ic<16>{}, tf_ic<0>{});
    }
}

static bool tf_q4k_weights_ok(const uint8_t* w, int nb, int col_bytes) {
    return w && ((uintptr_t)w & 15) == 0 && (col_bytes & 15) == 0 && col_bytes >= nb * 144;
}

static TfActSrc tf_src_q8(const int8_t* xq, const float* xd) {
    return TfActSrc{TF_SRC_Q8, xq, xd, nullptr, nullptr, 0.f};
}
static TfActSrc tf_src_f32(const float* x) {
    return TfActSrc{TF_SRC_F32, nullptr, nullptr, x, nullptr, 0.f};
}

static int tf_q4k_rows(const TfQ4kMats& m, const TfActSrc& src, int n_rows, int col_bytes,
                       int use_bias, int use_res, const float* residual, tf_stream_t stream) {
    TF_CHECK_ARG(tf_src_ok(src));
    const int nb = n_rows / 256;
    const int n_total = m.n0 + m.n1 + m.n2;
    const int lds = tf_act_lds_bytes(nb, false);
    int rc = 0;
    if (src.kind == TF_SRC_Q8 && nb <= 8 && ((uintptr_t)src.xq & 15) == 0 &&
        ((uintptr_t)src.xd & 7) == 0) {
        // the lane map of tf_q4k_dispatch for nb <= 8: one part per lane
        auto go = [&](auto spr) {
            constexpr int SPR = decltype(spr)::value;
            auto fn = tf_q4k_rows_gq8_kernel<SPR, 1>;
            const int tasks = (n_total + 16 / SPR - 1) / (16 / SPR);
            const int BT = tf_block_threads(tf_bt_rows(SPR), tasks);
            const int blocks = tf_persistent_blocks((const void*)fn, BT, 0, tasks);
            hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), 0, tf_stream(stream), m, src.xq,
                               src.xd, nb, col_bytes, use_bias, use_res, residual);
            return (int)TF_LAUNCH_RESULT();
        };
        return nb <= 4 ? go(tf_ic<4>{}) : go(tf_ic<8>{});
    }
    tf_q4k_dispatch(nb, [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        auto fn = tf_sk_pick(src.kind, tf_q4k_rows_kernel<SPR, IT, TF_SRC_Q8>,
                             tf_q4k_rows_kernel<SPR, IT, TF_SRC_F32>,
                             tf_q4k_rows_kernel<SPR, IT, TF_SRC_NORM>,
                             tf_q4k_rows_kernel<SPR, IT, TF_SRC_FLASH>);
        const int tasks = (n_total + 16 / SPR - 1) / (16 / SPR);
        const int BT = tf_block_threads(tf_bt_rows(SPR, src.kind), tasks);
        const int blocks = tf_persistent_blocks((const void*)fn, BT, lds, tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), lds, tf_stream(stream), m, src, nb,
                           col_bytes, use_bias, use_res, residual);
        rc = TF_LAUNCH_RESULT();
    });
    return rc;
}

static int tf_q4k_pair_rows(const uint8_t* wa, const uint8_t* wb, const TfActSrc& src,
                            float* out_a, float* out_b, int n_rows, int n_cols, int col_bytes,
                            int mode, tf_stream_t stream) {
    TF_CHECK_ARG(tf_src_ok(src) && src.kind != TF_SRC_FLASH);
    const int nb = n_rows / 256;
    const int lds = tf_act_lds_bytes(nb, false);
    int rc = 0;
    tf_q4k_dispatch(nb, [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        auto fn = mode == 0 ? tf_sk_pick(src.kind, tf_q4k_pair_rows_kernel<SPR, IT, 0, TF_SRC_Q8>,
                                         tf_q4k_pair_rows_kernel<SPR, IT, 0, TF_SRC_F32>,
                                         tf_q4k_pair_rows_kernel<SPR, IT, 0, TF_SRC_NORM>)
                            : tf_sk_pick(src.kind, tf_q4k_pair_rows_kernel<SPR, IT, 1, TF_SRC_Q8>,
                                         tf_q4k_pair_rows_kernel<SPR, IT, 1, TF_SRC_F32>,
                                         tf_q4k_pair_rows_kernel<SPR, IT, 1, TF_SRC_NORM>);
        const int jpw = SPR <= 8 ? 16 / SPR / 2 : 1;
        const int tasks = (n_cols + jpw - 1) / jpw;
        const int BT = tf_block_threads(tf_bt_pair(SPR), tasks);
        const int blocks = tf_persistent_blocks((const void*)fn, BT, lds, tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), lds, tf_stream(stream), wa, wb, src, out_a,
                           out_b, nb, n_cols, col_bytes);
        rc = TF_LAUNCH_RESULT();
    });
    return rc;
}

// ---------------------------------------------------------------- C ABI

extern "C" int tf_gemv_q4k_q8(const uint8_t* w, const int8_t* xq, const float* xd,
                              float* out, int n_rows, int n_cols, int col_bytes,
                              int use_bias, const float* bias, int use_res,
                              const float* residual, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && tf_q4k_weights_ok(w, nb, col_bytes));
    TF_CHECK_ARG(xq && xd && out && (!use_bias || bias) && use_res >= 0 && use_res <= 2);
    TF_CHECK_ARG(use_res != 1 || residual);
    TfQ4kMats m{w, nullptr, nullptr, out, nullptr, nullptr, bias, nullptr, nullptr,
                n_cols, 0, 0};
    return tf_q4k_rows(m, tf_src_q8(xq, xd), n_rows, col_bytes, use_bias, use_res, residual, stream);
}

extern "C" int tf_gemv_q4k_flash_out(const uint8_t* w, const float* partial, int n_head,
                                     int head_dim, int n_split, float* out, int n_cols,
                                     int col_bytes, int use_res, float* attn_out,
                                     int8_t* attn_q8, float* attn_d8, tf_stream_t stream) {
    const int n_rows = n_head * head_dim;
    const int nb = n_rows / 256;
    TF_CHECK_ARG(n_head > 0 && n_head <= 32 && n_rows % 256 == 0 && n_rows <= 4096 && n_cols > 0);
    TF_CHECK_ARG(n_split >= 1 && n_split <= 64 && n_head * (n_split + 1) <= TF_FLASH_STAGE_W);
    TF_CHECK_ARG(tf_q4k_weights_ok(w, nb, col_bytes) && out && (use_res == 0 || use_res == 2));
    TfQ4kMats m{w, nullptr, nullptr, out, nullptr, nullptr, nullptr, nullptr, nullptr,
                n_cols, 0, 0};
    const TfActSrc src{TF_SRC_FLASH, nullptr, nullptr, partial, nullptr, 0.f, n_split, head_dim,
                       attn_out, attn_q8, attn_d8};
    return tf_q4k_rows(m, src, n_rows, col_bytes, 0, use_res, nullptr, stream);
}

extern "C" int tf_gemv_q4k_f32(const uint8_t* w, const float* x, float* out, int n_rows,
                               int n_cols, int col_bytes, int use_bias, const float* bias,
                               int use_res, const float* residual, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && tf_q4k_weights_ok(w, nb, col_bytes));
    TF_CHECK_ARG(x && out && (!use_bias || bias) && use_res >= 0 && use_res <= 2);
    TF_CHECK_ARG(use_res != 1 || residual);
    TfQ4kMats m{w, nullptr, nullptr, out, nullptr, nullptr, bias, nullptr, nullptr,
                n_cols, 0, 0};
    return tf_q4k_rows(m, tf_src_f32(x), n_rows, col_bytes, use_bias, use_res, residual, stream);
}

extern "C" int tf_gemv_q4k_pair(const uint8_t* wa, const uint8_t* wb, const int8_t* xq,
                                const float* xd, float* out_a, float* out_b, int n_rows,
                                int n_a, int n_b, int col_bytes, int use_bias,
                                const float* ba, const float* bb, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_a >= 0 && n_b >= 0 && n_a + n_b > 0);
    TF_CHECK_ARG(tf_q4k_weights_ok(wa, nb, col_bytes) && tf_q4k_weights_ok(wb, nb, col_bytes));
    TF_CHECK_ARG(xq && xd && out_a && out_b && (!use_bias || (ba && bb)));
    TfQ4kMats m{wa, wb, nullptr, out_a, out_b, nullptr, ba, bb, nullptr, n_a, n_b, 0};
    return tf_q4k_rows(m, tf_src_q8(xq, xd), n_rows, col_bytes, use_bias, 0, nullptr, stream);
}

extern "C" int tf_gemv_q4k_qkv(const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                               const int8_t* xq, const float* xd, float* q, float* k,
                               float* v, int n_rows, int n_q, int n_k, int n_v,
                               int col_bytes, int use_bias, const float* bq,
                               const float* bk, const float* bv, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_q >= 0 && n_k >= 0 && n_v >= 0 && n_q + n_k + n_v > 0);
    TF_CHECK_ARG(tf_q4k_weights_ok(wq, nb, col_bytes) && tf_q4k_weights_ok(wk, nb, col_bytes) &&
                 tf_q4k_weights_ok(wv, nb, col_bytes));
    TF_CHECK_ARG(xq && xd && q && k && v && (!use_bias || (bq && bk && bv)));
    TfQ4kMats m{wq, wk, wv, q, k, v, bq, bk, bv, n_q, n_k, n_v};
    return tf_q4k_rows(m, tf_src_q8(xq, xd), n_rows, col_bytes, use_bias, 0, nullptr, stream);
}

extern "C" int tf_gemv_q4k_dual(const uint8_t* wa, const uint8_t* wb, const int8_t* xq,
                                const float* xd, float* out_a, float* out_b, int n_rows,
                                int n_cols, int col_bytes, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0);
    TF_CHECK_ARG(tf_q4k_weights_ok(wa, nb, col_bytes) && tf_q4k_weights_ok(wb, nb, col_bytes));
    TF_CHECK_ARG(xq && xd && out_a && out_b);
    return tf_q4k_pair_rows(wa, wb, tf_src_q8(xq, xd), out_a, out_b, n_rows, n_cols, col_bytes, 1,
                            stream);
}

extern "C" int tf_gemv_q4k_ffn(const uint8_t* gate, const uint8_t* up, const int8_t* xq,
                               const float* xd, float* out, int n_rows, int n_cols,
                               int col_bytes, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0);
    TF_CHECK_ARG(tf_q4k_weights_ok(gate, nb, col_bytes) && tf_q4k_weights_ok(up, nb, col_bytes));
    TF_CHECK_ARG(xq && xd && out);
    return tf_q4k_pair_rows(gate, up, tf_src_q8(xq, xd), out, nullptr, n_rows, n_cols, col_bytes, 0,
                            stream);
}

extern "C" int tf_gemv_q4k_ffn_f32(const uint8_t* gate, const uint8_t* up, const float* x,
                                   float* out, int n_rows, int n_cols, int col_bytes,
                                   tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0);
    TF_CHECK_ARG(tf_q4k_weights_ok(gate, nb, col_bytes) && tf_q4k_weights_ok(up, nb, col_bytes));
    TF_CHECK_ARG(x && out);
    return tf_q4k_pair_rows(gate, up, tf_src_f32(x), out, nullptr, n_rows, n_cols, col_bytes, 0,
                            stream);
}

extern "C" int tf_gemv_q4k_ffn_norm(const uint8_t* gate, const uint8_t* up, const float* x,
                                    const float* norm_w, float eps, float* out, int n_rows,
                                    int n_cols, int col_bytes, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0);
    TF_CHECK_ARG(tf_q4k_weights_ok(gate, nb, col_bytes) && tf_q4k_weights_ok(up, nb, col_bytes));
    TF_CHECK_ARG(x && norm_w && out);
    return tf_q4k_pair_rows(gate, up, TfActSrc{TF_SRC_NORM, nullptr, nullptr, x, norm_w, eps, n_rows}, out,
                            nullptr, n_rows, n_cols, col_bytes, 0, stream);
}

extern "C" int tf_gemv_q4k_q8_splitk(const uint8_t* w, const int8_t* xq, const float* xd,
                                     float* partial, int n_rows, int n_cols, int col_bytes,
                                     int n_split, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && n_split >= 1 && n_split <= 8);
    TF_CHECK_ARG(tf_q4k_weights_ok(w, nb, col_bytes) && xq && xd && partial);
    const int lds = tf_act_lds_bytes(nb, false);
    const int len = (nb + n_split - 1) / n_split;
    int rc = 0;
    tf_q4k_dispatch(len, [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        auto fn = tf_q4k_splitk_kernel<SPR, IT>;
        const long long total = (long long)n_split * n_cols;
        const int tasks = (int)((total + 16 / SPR - 1) / (16 / SPR));
        const int blocks = tf_persistent_blocks((const void*)fn, 256, lds, tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), lds, tf_stream(stream), w,
                           tf_src_q8(xq, xd), partial, nb, n_cols, col_bytes, n_split);
        rc = TF_LAUNCH_RESULT();
    });
    return rc;
}

extern "C" int tf_gemv_splitk_reduce(const float* partial, float* out, int n_cols,
                                     int n_split, int use_bias, const float* bias,
                                     int use_res, const float* residual, tf_stream_t stream) {
    TF_CHECK_ARG(partial && out && n_cols > 0 && n_split >= 1);
    TF_CHECK_ARG((!use_bias || bias) && use_res >= 0 && use_res <= 2 && (use_res != 1 || residual));
    hipLaunchKernelGGL(tf_splitk_reduce_kernel, dim3((n_cols + 255) / 256), dim3(256), 0,
                       tf_stream(stream), partial, out, n_cols, n_split, use_bias, bias,
                       use_res, residual);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_q4k_block_dots(const uint8_t* w, const int8_t* xq, int32_t* dots,
                                 int32_t* sums, int n_rows, int n_cols, int col_bytes,
                                 tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && tf_q4k_weights_ok(w, nb, col_bytes));
    TF_CHECK_ARG(xq && ((uintptr_t)xq & 15) == 0 && dots && sums);
    const long long total = (long long)n_cols * nb * 4;
    const int lds = TF_Q8_LDS_BYTES(nb) + nb * 8 * 4;
    hipLaunchKernelGGL(tf_q4k_block_dots_kernel, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), lds, tf_stream(stream), w, xq, dots, sums, nb, n_cols,
                       col_bytes);
    return TF_LAUNCH_RESULT();
}
