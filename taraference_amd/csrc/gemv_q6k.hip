// Q6_K GEMV family for gfx950 (batch 1).
//
// Replaces kernels/gemv.cu gemv_q6_k_compact_global (:515),
// gemv_q6_k_compact_global_{4way,8way} (:2025, :2081),
// gemv_q6_k_compact_global_splitk (:1998), gemv_q6_k (:405) and the load-time
// repack cuda/load.rs:145-159.
//
// The reference splits a tall Q6_K row over 4 or 8 warps of one block and
// merges in shared memory.  Here a row is spread over 16 four-lane slots of
// one wave with all of its weight loads issued up front, and the grid is
// persistent, so the tall ffn_down and the wide lm_head use the same kernel.
#include <type_traits>

#include "lds_dma.hpp"
#include "q6k.hpp"
#include "tf_host.hpp"

template <int SPR, int ITERS, int SK>
__global__ __launch_bounds__(tf_bt_rows(SPR)) void tf_q6k_rows_kernel(
    const uint8_t* __restrict__ w, TfActSrc src, float* __restrict__ out, int nb, int n_cols,
    int col_bytes, int use_bias, const float* __restrict__ bias, int use_res,
    const float* __restrict__ residual) {
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
    // A wide activation (16 super-blocks or more) is staged before the first
    // weight loads: issued after them, its loads would complete only behind
    // them (in issue order), and the staging would then lengthen the critical
    // path (Q6_K 11008 -> 2048: 7.6 -> 7.1 us back to back); a narrow one costs
    // less than the delay it would add to the weight stream.  (The
    // activation's loads issued first, the weight loads right behind them and
    // the image written after: 7.11 us, Q4_K 11008 -> 2048 5.57 vs 5.77 us,
    // within the run-to-run spread.)
    const bool act_first = nb >= 16;
    if (act_first) tf_stage_act<false, SK>(src, nb, lds);
    if (ITERS > 0 && task < n_tasks)
        tf_q6k_row_load<SPR, ITERS>(w + (size_t)(j < n_cols ? j : 0) * col_bytes, j < n_cols, 0,
                                    nb, sir, p, cur);
    if (!act_first) tf_stage_act<false, SK>(src, nb, lds);
    const TfAct x = tf_act_view(lds, nb);
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
            if (use_res == 1) acc += residual[j];
            else if (use_res == 2) acc += out[j];
            if (use_bias) acc += bias[j];
            out[j] = acc;
        }
        if constexpr (ITERS > 0) cur = nxt;
        j = jn;
    }
}

// Wide Q6_K GEMV fed by HBM -> LDS copies (the lm_head: K = 2048, 151936
// rows, 256 MB per launch).  Each of the 8 waves of a workgroup owns an
// S-slot LDS ring and streams its tasks (R consecutive rows, one contiguous
// run of R * NB * 212 bytes) into it with global_load_lds_dwordx4, S - 1
// tasks in flight while one computes, so the wave's memory queue never waits
// on its own arithmetic.  Lanes: 64 / R per row (row r = lane / (64 / R));
// lane u of a row takes parts (sb, p) = (u / 4 + (16 / R) i, u % 4).  The
// row's lanes are summed with one group reduction.  Same integer stage and
// scaling as tf_q6k_part_dot.
template <int NB, int R, int S>
struct TfQ6Dma {
    static constexpr int CHUNKS = R * NB * 212 / 16;  // 16-byte chunks per task
    static constexpr int NI = (CHUNKS + 63) / 64;     // copy instructions per task
    static constexpr int SLOT = NI * 1024;            // bytes per ring slot
    static constexpr int LPR = 64 / R;                // lanes per row
    static constexpr int UPL = NB * 4 / LPR;          // (super-block, part) units per lane
    static_assert(R == 1 || R == 2 || R == 4, "rows per task");
    static_assert(NB % 4 == 0 && UPL >= 1 && UPL * LPR == NB * 4, "lane map");
    static constexpr int LDS = 8 * S * SLOT;          // the rings of the 8 waves
};

// Copies of task `task` into the slot at LDS byte slot_off: copy i of lane l
// moves bytes [16 c, 16 c + 16) of the task's run, c = 64 i + l; chunks past
// the run (or past the matrix) copy the run's first bytes into LDS bytes
// nothing reads.
template <int NB, int R, int S>
__device__ __forceinline__ void tf_q6d_issue(const uint8_t* __restrict__ w, int n_cols,
                                             int task, uint32_t slot_off, int lane) {
    using D = TfQ6Dma<NB, R, S>;
    const uint8_t* base = w + (size_t)task * (R * NB * 212);
    const int left = (n_cols - task * R) * (NB * 212 / 16);  // chunks inside the matrix
#pragma unroll
    for (int i = 0; i < D::NI; i++) {
        const int c = 64 * i + lane;
        tf_lds_dma16(c < D::CHUNKS && c < left ? base + 16 * c : base, slot_off + 1024 * i);
    }
}

template <int NB, int R, int S, int SK>
__global__ __launch_bounds__(512) void tf_q6k_dma_rows_kernel(
    const uint8_t* __restrict__ w, TfActSrc src, float* __restrict__ out, int n_cols,
    int col_bytes) {
    using D = TfQ6Dma<NB, R, S>;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int act = (tf_act_lds_bytes(NB, false) + 15) & ~15;
    uint8_t* ring = lds + act + wave * S * D::SLOT;
    const uint32_t ring_off = tf_lds_off(ring);
    const int n_tasks = (n_cols + R - 1) / R;
    const int G = gridDim.x * 8;
    const int g = wave * gridDim.x + blockIdx.x;  // this wave's first task
    // the first S - 1 tasks in flight (wave 0 stages the activation first: its
    // staging loads would otherwise wait behind its copies)
    if (wave != 0) {
#pragma unroll
        for (int q = 0; q < S - 1; q++)
            if (g + q * G < n_tasks)
                tf_q6d_issue<NB, R, S>(w, n_cols, g + q * G, ring_off + q * D::SLOT, lane);
    }
    tf_stage_act<false, SK>(src, NB, lds);
    if (wave == 0) {
#pragma unroll
        for (int q = 0; q < S - 1; q++)
            if (g + q * G < n_tasks)
                tf_q6d_issue<NB, R, S>(w, n_cols, g + q * G, ring_off + q * D::SLOT, lane);
    }
    const TfAct x = tf_act_view(lds, NB);
    const int r = lane / D::LPR, u = lane % D::LPR, p = u & 3, n = p >> 1, h = p & 1;
    int k = 0;
    for (int task = g; task < n_tasks; task += G) {
        // refill: task + (S - 1) G goes to the slot freed by the previous task
        if (task + (S - 1) * G < n_tasks)
            tf_q6d_issue<NB, R, S>(w, n_cols, task + (S - 1) * G,
                                   ring_off + (k == 0 ? S - 1 : k - 1) * D::SLOT, lane);
        // this task's copies have landed: at most the S - 1 later tasks' are pending
        if (task + (S - 1) * G < n_tasks)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 1) * D::NI) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const uint8_t* rowp = ring + k * D::SLOT + r * (NB * 212);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < D::UPL; i++) {
            const int sb = (u >> 2) + (D::LPR / 4) * i;
            // a block is 4-byte aligned in LDS (212 = 4 * 53)
            const uint32_t* blk = reinterpret_cast<const uint32_t*>(rowp + sb * 212);
            TfQ6kPart q;
            const uint32_t* pa = blk + 16 * n + 4 * h;
            const uint32_t* ph = blk + 32 + 8 * n + 4 * h;
            q.a = tf_u32x4{pa[0], pa[1], pa[2], pa[3]};
            q.b = tf_u32x4{pa[8], pa[9], pa[10], pa[11]};
            q.hq = tf_u32x4{ph[0], ph[1], ph[2], ph[3]};
            q.sc = tf_u32x2{blk[48 + 2 * n], blk[49 + 2 * n]};
            q.d = blk[52];
            acc += tf_q6k_part_dot(q, p, sb, x);
        }
        acc = tf_group_sum<D::LPR>(acc);
        const int j = task * R + r;
        if (u == 0 && j < n_cols) out[j] = acc;
        // the slot's reads are done before the next iteration refills it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        k = k + 1 == S ? 0 : k + 1;
    }
}

template <int SPR, int ITERS>
__global__ __launch_bounds__(256) void tf_q6k_splitk_kernel(
    const uint8_t* __restrict__ w, TfActSrc src, float* __restrict__ partial, int nb,
    int n_cols, int col_bytes, int n_split) {
    extern __shared__ __align__(16) uint8_t lds[];
    tf_stage_act<false, TF_SRC_Q8>(src, nb, lds);
    const TfAct x = tf_act_view(lds, nb);
    constexpr int UNITS = 16 / SPR;
    const int lane = threadIdx.x & 63;
    const int p = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
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
            TfQ6kRow<ITERS> rr;
            tf_q6k_row_load<SPR, ITERS>(col, valid, sb0, sb1, sir, p, rr);
            acc = tf_q6k_row_partial<SPR, ITERS>(rr, valid, sb0, sb1, sir, p, x);
        } else {
            acc = tf_q6k_row_partial_loop<SPR>(col, valid, sb0, sb1, sir, p, x);
        }
        acc = tf_group_sum<4 * SPR>(acc);
        if (valid && (lane & (4 * SPR - 1)) == 0) partial[(size_t)s * n_cols + j] = acc;
    }
}

// f32 activation over raw 210-byte blocks (kernels/gemv.cu:405-438).  x and
// its 16-value sums live in LDS; per scale group the lane forms
// sum(q*x) - 32*sum(x), then scales by d*sc.
template <int SPR>
__global__ __launch_bounds__(256) void tf_q6k_f32_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ xg, float* __restrict__ out,
    int nb, int n_cols, int col_bytes, int use_bias, const float* __restrict__ bias,
    int use_res, const float* __restrict__ residual) {
    extern __shared__ __align__(16) uint8_t lds[];
    float* xs = reinterpret_cast<float*>(lds);
    float* xsum = xs + nb * 256;
    for (int i = threadIdx.x; i < nb * 16; i += blockDim.x) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 16; k += 4) {
            const float4 v = *reinterpret_cast<const float4*>(xg + i * 16 + k);
            *reinterpret_cast<float4*>(xs + i * 16 + k) = v;
            s += (v.x + v.y) + (v.z + v.w);
        }
        xsum[i] = s;
    }
    __syncthreads();
    constexpr int UNITS = 16 / SPR;
    const int lane = threadIdx.x & 63;
    const int p = lane & 3, slot = lane >> 2, unit = slot / SPR, sir = slot % SPR;
    const int n = p >> 1, h = p & 1;
    const int wave = tf_wave_id();
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    for (int r0 = wave * UNITS; r0 < n_cols; r0 += nwaves * UNITS) {
        const int j = r0 + unit;
        const bool valid = j < n_cols;
        const uint8_t* col = w + (size_t)(valid ? j : 0) * col_bytes;
        float acc = 0.f;
        for (int sb = sir; valid && sb < nb; sb += SPR) {
            TfQ6kPart q;
            tf_q6k_load_r(col + (size_t)sb * 210, p, q);
            const float d = tf_h2f(q.d);
            float part = 0.f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float* xv = xs + sb * 256 + 128 * n + 32 * k + 16 * h;
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t word = tf_q6k_word(q, k, i);
                    const float4 xx = *reinterpret_cast<const float4*>(xv + 4 * i);
                    s += (float)(word & 0xff) * xx.x;
                    s += (float)((word >> 8) & 0xff) * xx.y;
                    s += (float)((word >> 16) & 0xff) * xx.z;
                    s += (float)(word >> 24) * xx.w;
                }
                s -= 32.f * xsum[sb * 16 + 8 * n + 2 * k + h];
                part += (float)tf_q6k_scale(q, p, k) * s;
            }
            acc += d * part;
        }
        acc = tf_group_sum<4 * SPR>(acc);
        if (valid && (lane & (4 * SPR - 1)) == 0) {
            if (use_res == 1) acc += residual[j];
            else if (use_res == 2) acc += out[j];
            if (use_bias) acc += bias[j];
            out[j] = acc;
        }
    }
}

template <int BLOCK_BYTES>
__global__ __launch_bounds__(256) void tf_q6k_block_dots_kernel(
    const uint8_t* __restrict__ w, const int8_t* __restrict__ xq, int32_t* __restrict__ dots,
    int nb, int n_cols, int col_bytes) {
    extern __shared__ __align__(16) uint8_t lds[];
    // stage only the bytes and 16-value sums (d8 is not part of the integer stage)
    int8_t* q8s = reinterpret_cast<int8_t*>(lds);
    int32_t* s16 = reinterpret_cast<int32_t*>(lds + TF_Q8_LDS_BYTES(nb));
    for (int i = threadIdx.x; i < nb * 16; i += blockDim.x) {
        const tf_u32x4 a = tf_ld16(xq + i * 16);
        *reinterpret_cast<tf_u32x4*>(q8s + tf_q8_pad(16 * i)) = a;
        const int one = 0x01010101;
        int s = tf_dot4(one, (int)a.x, 0);
        s = tf_dot4(one, (int)a.y, s);
        s = tf_dot4(one, (int)a.z, s);
        s = tf_dot4(one, (int)a.w, s);
        s16[i] = s;
    }
    __syncthreads();
    const long long task = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (task >= (long long)n_cols * nb * 4) return;
    const int p = (int)(task & 3);
    const long long blk = task >> 2;
    const int j = (int)(blk / nb), sb = (int)(blk % nb);
    TfQ6kPart q;
    const uint8_t* base = w + (size_t)j * col_bytes + (size_t)sb * BLOCK_BYTES;
    if (BLOCK_BYTES == 212) tf_q6k_load_c(base, p, q);
    else tf_q6k_load_r(base, p, q);
    int idot[4];
    tf_q6k_idots(q, p, q8s + sb * 320, s16 + sb * 16, idot);
    const int n = p >> 1, h = p & 1;
    for (int k = 0; k < 4; k++) dots[((size_t)j * nb + sb) * 16 + 8 * n + 2 * k + h] = idot[k];
}

__global__ __launch_bounds__(256) void tf_q6k_repack_kernel(const uint8_t* __restrict__ raw,
                                                             uint8_t* __restrict__ dst, int nb,
                                                             int n_cols, int col_bytes) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // dst dword
    const long long total = (long long)n_cols * nb * 53;
    if (i >= total) return;
    const long long blk = i / 53;
    const int k = (int)(i - blk * 53);
    const int j = (int)(blk / nb), sb = (int)(blk % nb);
    const uint8_t* src = raw + (size_t)j * col_bytes + (size_t)sb * 210 + 4 * k;
    const uint16_t* s2 = reinterpret_cast<const uint16_t*>(src);
    uint32_t v = s2[0];
    if (k < 52) v |= (uint32_t)s2[1] << 16;  // bytes 208,209 then two zero pad bytes
    reinterpret_cast<uint32_t*>(dst)[i] = v;
}

// ---------------------------------------------------------------- dispatch

template <int V>
using tf_ic6 = std::integral_constant<int, V>;

template <typename F>
static void tf_q6k_dispatch(int len, F&& f) {
    if (len <= 4) return f(tf_ic6<4>{}, tf_ic6<1>{});
    if (len <= 8) return f(tf_ic6<8>{}, tf_ic6<1>{});
    switch ((len + 15) / 16) {
    case 1: return f(tf_ic6<16>{}, tf_ic6<1>{});
    case 2: return f(tf_ic6<16>{}, tf_ic6<2>{});
    case 3: return f(tf_ic6<16>{}, tf_ic6<3>{});
    case 4: return f(tf_ic6<16>{}, tf_ic6<4>{});
    case 5: return f(tf_ic6<16>{}, tf_ic6<5>{});
    default: return f(tf_ic6<16>{}, tf_ic6<0>{});
    }
}

static bool tf_q6c_weights_ok(const uint8_t* w, int nb, int col_bytes) {
    return w && ((uintptr_t)w & 3) == 0 && (col_bytes & 3) == 0 && col_bytes >= nb * 212;
}

// The LDS-fed kernel serves wide matrices with K = 1024 or 2048, 16-byte
// aligned rows of exactly nb compact blocks, a Q8 activation and a plain output.
static bool tf_q6k_dma_ok(const uint8_t* w, int nb, int n_cols, int col_bytes, int use_bias,
                          int use_res) {
    return (nb == 8 || nb == 4) && col_bytes == nb * 212 && ((uintptr_t)w & 15) == 0 &&
           n_cols >= 65536 && !use_bias && use_res == 0;
}

static int tf_q6k_rows(const uint8_t* w, const TfActSrc& src, float* out, int n_rows,
                       int n_cols, int col_bytes, int use_bias, const float* bias, int use_res,
                       const float* residual, tf_stream_t stream) {
    TF_CHECK_ARG(tf_src_ok(src) && src.kind != TF_SRC_FLASH);
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && tf_q6c_weights_ok(w, nb, col_bytes));
    TF_CHECK_ARG(out && (!use_bias || bias) && use_res >= 0 && use_res <= 2);
    TF_CHECK_ARG(use_res != 1 || residual);
    TF_CHECK_ARG(src.kind == TF_SRC_Q8 ? (src.xq && src.xd) : (src.x != nullptr));
    const int lds = tf_act_lds_bytes(nb, false);
    int rc = 0;
    if (src.kind == TF_SRC_Q8 && tf_q6k_dma_ok(w, nb, n_cols, col_bytes, use_bias, use_res)) {
        auto go = [&](auto nbc, auto rc_, auto sc_) {
            constexpr int NB = decltype(nbc)::value, R = decltype(rc_)::value,
                          S = decltype(sc_)::value;
            auto fn = tf_q6k_dma_rows_kernel<NB, R, S, TF_SRC_Q8>;
            const int bytes = ((tf_act_lds_bytes(NB, false) + 15) & ~15) + TfQ6Dma<NB, R, S>::LDS;
            if (tf_set_lds_limit((const void*)fn, bytes) != 0) return (int)hipErrorInvalidValue;
            hipLaunchKernelGGL(fn, dim3(tf_device_cus()), dim3(512), bytes, tf_stream(stream), w,
                               src, out, n_cols, col_bytes);
            return (int)TF_LAUNCH_RESULT();
        };
        // four rows per task, two ring slots per wave (measured on the 3B
        // lm_head against 2 rows x 3 or 4 slots and register-staged copies)
        if (nb == 4) return go(tf_ic6<4>{}, tf_ic6<4>{}, tf_ic6<2>{});
        return go(tf_ic6<8>{}, tf_ic6<4>{}, tf_ic6<2>{});
    }
    tf_q6k_dispatch(nb, [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        auto fn = tf_sk_pick(src.kind, tf_q6k_rows_kernel<SPR, IT, TF_SRC_Q8>,
                             tf_q6k_rows_kernel<SPR, IT, TF_SRC_F32>,
                             tf_q6k_rows_kernel<SPR, IT, TF_SRC_NORM>);
        const int tasks = (n_cols + 16 / SPR - 1) / (16 / SPR);
        const int BT = tf_block_threads(tf_bt_rows(SPR), tasks);
        const int blocks = tf_persistent_blocks((const void*)fn, BT, lds, tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(BT), lds, tf_stream(stream), w, src, out, nb,
                           n_cols, col_bytes, use_bias, bias, use_res, residual);
        rc = TF_LAUNCH_RESULT();
    });
    return rc;
}

// ---------------------------------------------------------------- C ABI

extern "C" int tf_gemv_q6k_compact_q8(const uint8_t* w, const int8_t* xq, const float* xd,
                                      float* out, int n_rows, int n_cols, int col_bytes,
                                      int use_bias, const float* bias, int use_res,
                                      const float* residual, tf_stream_t stream) {
    return tf_q6k_rows(w, TfActSrc{TF_SRC_Q8, xq, xd, nullptr, nullptr, 0.f}, out, n_rows, n_cols,
                       col_bytes, use_bias, bias, use_res, residual, stream);
}

extern "C" int tf_gemv_q6k_down_splitk(const uint8_t* w, const int8_t* xq, const float* xd,
                                       float* out, int n_rows, int n_cols, int col_bytes,
                                       int use_bias, const float* bias, int use_res,
                                       const float* residual, tf_stream_t stream) {
    // Full-K per row inside one wave: the reference's in-block 4/8-way merge
    // collapses into the wave reduction.
    return tf_q6k_rows(w, TfActSrc{TF_SRC_Q8, xq, xd, nullptr, nullptr, 0.f}, out, n_rows, n_cols,
                       col_bytes, use_bias, bias, use_res, residual, stream);
}

extern "C" int tf_gemv_q6k_compact_q8_splitk(const uint8_t* w, const int8_t* xq,
                                             const float* xd, float* partial, int n_rows,
                                             int n_cols, int col_bytes, int n_split,
                                             tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && n_split >= 1 && n_split <= 8);
    TF_CHECK_ARG(tf_q6c_weights_ok(w, nb, col_bytes) && xq && xd && partial);
    const int lds = tf_act_lds_bytes(nb, false);
    int rc = 0;
    tf_q6k_dispatch((nb + n_split - 1) / n_split, [&](auto spr, auto it) {
        constexpr int SPR = decltype(spr)::value, IT = decltype(it)::value;
        auto fn = tf_q6k_splitk_kernel<SPR, IT>;
        const long long total = (long long)n_split * n_cols;
        const int tasks = (int)((total + 16 / SPR - 1) / (16 / SPR));
        const int blocks = tf_persistent_blocks((const void*)fn, 256, lds, tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), lds, tf_stream(stream), w,
                           TfActSrc{TF_SRC_Q8, xq, xd, nullptr, nullptr, 0.f}, partial, nb, n_cols,
                           col_bytes, n_split);
        rc = TF_LAUNCH_RESULT();
    });
    return rc;
}

extern "C" int tf_gemv_q6k_f32(const uint8_t* w, const float* x, float* out, int n_rows,
                               int n_cols, int col_bytes, int use_bias, const float* bias,
                               int use_res, const float* residual, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && w && ((uintptr_t)w & 1) == 0 && (col_bytes & 1) == 0);
    TF_CHECK_ARG(col_bytes >= nb * 210 && x && ((uintptr_t)x & 15) == 0 && out);
    TF_CHECK_ARG((!use_bias || bias) && use_res >= 0 && use_res <= 2 && (use_res != 1 || residual));
    const int lds = nb * 256 * 4 + nb * 16 * 4;
    int rc = 0;
    auto go = [&](auto spr) {
        constexpr int SPR = decltype(spr)::value;
        auto fn = tf_q6k_f32_kernel<SPR>;
        const int tasks = (n_cols + 16 / SPR - 1) / (16 / SPR);
        const int blocks = tf_persistent_blocks((const void*)fn, 256, lds, tasks);
        hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), lds, tf_stream(stream), w, x, out, nb,
                           n_cols, col_bytes, use_bias, bias, use_res, residual);
        rc = TF_LAUNCH_RESULT();
    };
    if (nb <= 4) go(tf_ic6<4>{});
    else if (nb <= 8) go(tf_ic6<8>{});
    else go(tf_ic6<16>{});
    return rc;
}

extern "C" int tf_q6k_compact_repack(const uint8_t* raw, uint8_t* dst, int n_rows, int n_cols,
                                     int col_bytes, tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && raw && dst && ((uintptr_t)raw & 1) == 0);
    TF_CHECK_ARG((col_bytes & 1) == 0 && col_bytes >= nb * 210 && ((uintptr_t)dst & 3) == 0);
    const long long total = (long long)n_cols * nb * 53;
    hipLaunchKernelGGL(tf_q6k_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, tf_stream(stream), raw, dst, nb, n_cols, col_bytes);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_q6k_block_dots(const uint8_t* w, int block_bytes, const int8_t* xq,
                                 int32_t* dots, int n_rows, int n_cols, int col_bytes,
                                 tf_stream_t stream) {
    const int nb = n_rows / 256;
    TF_CHECK_ARG(nb > 0 && n_cols > 0 && w && xq && ((uintptr_t)xq & 15) == 0 && dots);
    TF_CHECK_ARG(block_bytes == 210 || block_bytes == 212);
    TF_CHECK_ARG(col_bytes >= nb * block_bytes);
    if (block_bytes == 212) TF_CHECK_ARG(tf_q6c_weights_ok(w, nb, col_bytes));
    else TF_CHECK_ARG(((uintptr_t)w & 1) == 0 && (col_bytes & 1) == 0);
    const long long total = (long long)n_cols * nb * 4;
    const int lds = TF_Q8_LDS_BYTES(nb) + nb * 64;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (block_bytes == 212)
        hipLaunchKernelGGL(tf_q6k_block_dots_kernel<212>, grid, dim3(256), lds,
                           tf_stream(stream), w, xq, dots, nb, n_cols, col_bytes);
    else
        hipLaunchKernelGGL(tf_q6k_block_dots_kernel<210>, grid, dim3(256), lds,
                           tf_stream(stream), w, xq, dots, nb, n_cols, col_bytes);
    return TF_LAUNCH_RESULT();
}
