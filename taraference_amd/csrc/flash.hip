// Split-KV flash decode for gfx950 (one query token).  head_dim 128 runs on
// the DMA-fed matrix-core partial further down; the vector-ALU kernel below
// serves head_dim 64 and 256.
//
// Replaces kernels/attn/flash.cu attn_flash_partial (:16), attn_flash_partial_d
// (:119) and attn_flash_reduce (:222).  The partial buffer keeps the
// reference layout partial[(h*n_split + s)*(2+hd)] = (m, l, O[hd]).
//
// A workgroup serves one (kv head, split) pair and every GQA query head that
// reads that kv head (G = n_head/n_kv), so each K/V byte of the split is read
// once.  Wave w owns heads w*HPW .. w*HPW+HPW-1.  The split is walked in
// 64-token tiles:
//   load:    the workgroup copies the K and V tiles to LDS with 16-byte
//            loads; the next tile is already in flight (registers) while the
//            current one is being used;
//   scores:  lane = token; K row from LDS (rows padded by 16 bytes so 16
//            lanes hit 16 distinct bank quads), q broadcast from LDS;
//   softmax: per head, wave max / sum with the running (m, l) rescale;
//   PV:      lane = head_dim/64 contiguous dims, exp weights broadcast from
//            LDS, V row from LDS.
// Each wave owns whole heads, so (m, l, O) is written without a merge.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "lds_dma.hpp"
#include "tf_common.hpp"
#include "tf_host.hpp"

#define TF_FLASH_TILE 64
#define TF_NEG_BIG (-1e30f)

template <int HD>
struct TfFlashLds {
    static constexpr int KROW = HD + 8;  // halves per padded K row
    static constexpr int CHUNKS = TF_FLASH_TILE * HD / 8;  // 16-byte chunks per tile
    static constexpr int PER_THREAD = CHUNKS / 256;
};

template <int HD, int HPW>
__global__ __launch_bounds__(256) void tf_flash_partial_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, float* __restrict__ partial, int n_head, int n_kv,
    int pos0, const int* __restrict__ pos0_dev, int n_split, float scale) {
    using L = TfFlashLds<HD>;
    constexpr int GMAX = 4 * HPW;
    constexpr int DPL = HD / 64;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    float* q_lds = reinterpret_cast<float*>(lds_raw);                      // [GMAX][HD]
    float* p_lds = q_lds + GMAX * HD;                                       // [GMAX][TILE]
    uint16_t* k_lds = reinterpret_cast<uint16_t*>(p_lds + GMAX * TF_FLASH_TILE);  // [TILE][KROW]
    uint16_t* v_lds = k_lds + TF_FLASH_TILE * L::KROW;                      // [TILE][HD]

    const int kv_h = blockIdx.x;
    const int s = blockIdx.y;
    const int G = n_head / n_kv;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int stride = n_kv * HD;
    if (pos0_dev) pos0 = pos0_dev[0];
    const int seq_len = pos0 + 1;
    const int chunk = (seq_len + n_split - 1) / n_split;
    const int t_begin = s * chunk;
    const int t_end = min(t_begin + chunk, seq_len);

    const uint16_t* kbase = k_cache + (size_t)kv_h * HD;
    const uint16_t* vbase = v_cache + (size_t)kv_h * HD;

    // tile t0 -> registers (row r of chunk c: r = c / (HD/8), col = 8*(c % (HD/8)))
    tf_u32x4 kr[L::PER_THREAD], vr[L::PER_THREAD];
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int i = 0; i < L::PER_THREAD; i++) {
            const int c = tid + 256 * i;
            const int r = c / (HD / 8), col = 8 * (c % (HD / 8));
            const int t = t0 + r;
            if (t < t_end) {
                kr[i] = tf_ld16(kbase + (size_t)t * stride + col);
                vr[i] = tf_ld16(vbase + (size_t)t * stride + col);
            } else {
                kr[i] = tf_u32x4{0, 0, 0, 0};
                vr[i] = tf_u32x4{0, 0, 0, 0};
            }
        }
    };
    if (t_begin < t_end) load_tile(t_begin);

    const float* qk = q + (size_t)kv_h * G * HD;
    for (int i = tid; i < GMAX * HD; i += 256) q_lds[i] = (i / HD) < G ? qk[i] : 0.f;

    float m[HPW], l[HPW], o[HPW][DPL];
#pragma unroll
    for (int hh = 0; hh < HPW; hh++) {
        m[hh] = TF_NEG_BIG;
        l[hh] = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; i++) o[hh][i] = 0.f;
    }

    for (int t0 = t_begin; t0 < t_end; t0 += TF_FLASH_TILE) {
        __syncthreads();  // previous tile fully consumed
#pragma unroll
        for (int i = 0; i < L::PER_THREAD; i++) {
            const int c = tid + 256 * i;
            const int r = c / (HD / 8), col = 8 * (c % (HD / 8));
            *reinterpret_cast<tf_u32x4*>(k_lds + r * L::KROW + col) = kr[i];
            *reinterpret_cast<tf_u32x4*>(v_lds + r * HD + col) = vr[i];
        }
        if (t0 + TF_FLASH_TILE < t_end) load_tile(t0 + TF_FLASH_TILE);
        __syncthreads();

        // ---- scores: lane = token
        const int t = t0 + lane;
        const bool tv = t < t_end;
        float sc[HPW];
#pragma unroll
        for (int hh = 0; hh < HPW; hh++) sc[hh] = 0.f;
        const uint16_t* krow = k_lds + lane * L::KROW;
#pragma unroll 4
        for (int d = 0; d < HD; d += 8) {
            const tf_u32x4 kw = *reinterpret_cast<const tf_u32x4*>(krow + d);
            float kf[8];
            kf[0] = tf_h2f(kw.x);
            kf[1] = tf_h2f(kw.x >> 16);
            kf[2] = tf_h2f(kw.y);
            kf[3] = tf_h2f(kw.y >> 16);
            kf[4] = tf_h2f(kw.z);
            kf[5] = tf_h2f(kw.z >> 16);
            kf[6] = tf_h2f(kw.w);
            kf[7] = tf_h2f(kw.w >> 16);
#pragma unroll
            for (int hh = 0; hh < HPW; hh++) {
                const float* qh = q_lds + (wave * HPW + hh) * HD + d;
                const float4 q0 = *reinterpret_cast<const float4*>(qh);
                const float4 q1 = *reinterpret_cast<const float4*>(qh + 4);
                float a = sc[hh];
                a += q0.x * kf[0];
                a += q0.y * kf[1];
                a += q0.z * kf[2];
                a += q0.w * kf[3];
                a += q1.x * kf[4];
                a += q1.y * kf[5];
                a += q1.z * kf[6];
                a += q1.w * kf[7];
                sc[hh] = a;
            }
        }
        // ---- online softmax per head (wave-uniform control flow)
        float alpha[HPW];
#pragma unroll
        for (int hh = 0; hh < HPW; hh++) {
            const float sv = tv ? sc[hh] * scale : TF_NEG_BIG;
            const float mx = tf_wave_max(sv);
            const float m_new = fmaxf(m[hh], mx);
            alpha[hh] = __expf(m[hh] - m_new);
            const float e = tv ? __expf(sv - m_new) : 0.f;
            p_lds[(wave * HPW + hh) * TF_FLASH_TILE + lane] = e;
            l[hh] = l[hh] * alpha[hh] + tf_group_sum<64>(e);
            m[hh] = m_new;
#pragma unroll
            for (int i = 0; i < DPL; i++) o[hh][i] *= alpha[hh];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // ---- PV: lane = DPL dims
        const int tlen = min(TF_FLASH_TILE, t_end - t0);
        const uint16_t* vcol = v_lds + lane * DPL;
        for (int tt = 0; tt < tlen; tt += 4) {
            float pw[HPW][4];
#pragma unroll
            for (int hh = 0; hh < HPW; hh++) {
                const float4 pv =
                    *reinterpret_cast<const float4*>(p_lds + (wave * HPW + hh) * TF_FLASH_TILE + tt);
                pw[hh][0] = pv.x;
                pw[hh][1] = pv.y;
                pw[hh][2] = pv.z;
                pw[hh][3] = pv.w;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint16_t* vr2 = vcol + (tt + u) * HD;
                float vf[DPL];
                if constexpr (DPL == 1) {
                    vf[0] = tf_h2f(vr2[0]);
                } else if constexpr (DPL == 2) {
                    const uint32_t vv = *reinterpret_cast<const uint32_t*>(vr2);
                    vf[0] = tf_h2f(vv);
                    vf[1] = tf_h2f(vv >> 16);
                } else {
                    const tf_u32x2 vv = *reinterpret_cast<const tf_u32x2*>(vr2);
                    vf[0] = tf_h2f(vv.x);
                    vf[1] = tf_h2f(vv.x >> 16);
                    vf[2] = tf_h2f(vv.y);
                    vf[3] = tf_h2f(vv.y >> 16);
                }
#pragma unroll
                for (int hh = 0; hh < HPW; hh++)
#pragma unroll
                    for (int i = 0; i < DPL; i++) o[hh][i] += pw[hh][u] * vf[i];
            }
        }
    }

    // ---- write (m, l, O) of this wave's heads
    const int po = 2 + HD;
#pragma unroll
    for (int hh = 0; hh < HPW; hh++) {
        const int g = wave * HPW + hh;
        if (g < G) {
            float* base = partial + ((size_t)(kv_h * G + g) * n_split + s) * po;
            if (lane == 0) {
                base[0] = m[hh];
                base[1] = l[hh];
            }
#pragma unroll
            for (int i = 0; i < DPL; i++) base[2 + lane * DPL + i] = o[hh][i];
        }
    }
}

typedef float tf_f32x4m __attribute__((ext_vector_type(4)));

// ------------------------------------------- matrix-core partial, DMA-fed
//
// head_dim 128, G <= 16.  The same split / (m, l, O) contract as the
// kernels above, shaped so that a workgroup keeps its whole split in
// flight and its waves never wait for each other while streaming: each of
// the 8 waves owns the 16-token tiles j = wave, wave + 8, ... of the split
// and moves them HBM -> LDS itself with global_load_lds_dwordx4 (1 KB per
// instruction, no register staging) into a private two-slot ring.  Only
// the query (copied once into LDS) and the final combine of the eight
// waves' (m, l, O) use workgroup barriers.  A 256-token split is one
// 128 KB burst per workgroup, issued before the first score is formed.
//
// Per tile and wave (lane l, n = l % 16, g = l / 16), on
// v_mfma_f32_16x16x32_f16 (A[n][8g .. 8g+7], B[8g .. 8g+7][n],
// C[4g + r][n]):
//   QK  S^T[token][head] = K Q^T: A = K row n (token t0 + n), one 16-byte
//       LDS read per k step; k step jj of lane group g covers dims
//       32 g + 8 jj .. +7 (a permutation of the 128 dims, applied to q
//       alike).  q is split into three f16 parts after a power-of-two
//       scale, K is f16: the products are exact.
//   softmax: a lane holds the scores of head n for tokens 4g .. 4g+3; the
//       head's maximum is a lane max plus two xor-shuffles (16, 32); each
//       lane keeps its own share of l, summed over the lane groups at the
//       end; p = e^(s - m) is split into two f16 parts (2^-22).
//   PV  O^T[dim][head] += V^T P^T with k = (token, part): k = 8g + i is the
//       hi part of token 4g + i for i < 4 and the lo part of token
//       4g + i - 4 otherwise, so B is the lane's own (hi, lo) p values and
//       A repeats the lane's four V values of dim 16 db + n; one MFMA per
//       16 dims covers both parts.  The accumulators hold head n only, so
//       the rescale by alpha is per lane.
// LDS: a K row's 16-byte chunk c sits at chunk c ^ (row % 16) (the DMA's
// source addresses are permuted, its LDS side stays linear), so the 16
// rows read by one lane group hit distinct banks; V rows go in blocks of
// four with 32 bytes of padding between blocks, so the four lane groups'
// column reads (rows 4g + i) fall in distinct banks and every V address is
// a per-lane base plus an immediate.
#define TF_FD_WAVES 8
#define TF_FD_TILE 16
#define TF_FD_VBLK 1056                        // 4 V rows + 32 bytes of padding
#define TF_FD_SLOT (4096 + 4 * TF_FD_VBLK)     // K (16 rows) + V (4 blocks)
#define TF_FD_WAVE (2 * TF_FD_SLOT)            // two-slot ring of one wave
#define TF_FD_Q (TF_FD_WAVES * TF_FD_WAVE)     // q block [16 heads][128] fp32
#define TF_FD_LDS (TF_FD_Q + 16 * 128 * 4)
#define TF_FD_CR 132                           // combine row: m, l, pad, O[128]

#ifdef TF_FLASH_STAMPS
__device__ unsigned long long tf_fd_stamps[4096 * 8];
extern "C" int tf_flash_debug_fd_stamps(unsigned long long* host) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(tf_fd_stamps), sizeof(tf_fd_stamps));
}
#define TF_FD_STAMP(k) st_[k] = __builtin_amdgcn_s_memrealtime()
#else
#define TF_FD_STAMP(k) \
    do {               \
    } while (0)
#endif

// With out != nullptr (n_split == 1 only) the workgroup's (m, l, O) is the
// whole context's: it writes out = O / max(l, 1e-20) (the merge of a single
// partition, bit-identical to tf_flash_reduce_kernel's) and, with q8, its
// Q8 instead of the partial, so the decode needs no second launch.
__global__ __launch_bounds__(512) void tf_flash_partial_dma_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, float* __restrict__ partial, int n_head, int n_kv,
    int pos0, const int* __restrict__ pos0_dev, int n_split, float scale,
    float* __restrict__ out, int8_t* __restrict__ q8, float* __restrict__ d8) {
    constexpr int HD = 128;
    extern __shared__ __align__(16) uint8_t lds_raw[];
#ifdef TF_FLASH_STAMPS
    unsigned long long st_[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#endif
    TF_FD_STAMP(0);
    const int kv_h = blockIdx.x, s = blockIdx.y;
    const int G = n_head / n_kv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int stride = n_kv * HD;
    if (pos0_dev) pos0 = pos0_dev[0];
    const int seq_len = pos0 + 1;
    const int chunk = (seq_len + n_split - 1) / n_split;
    const int t_begin = s * chunk;
    const int t_end = min(t_begin + chunk, seq_len);
    const int n_tiles = t_end > t_begin ? (t_end - t_begin + TF_FD_TILE - 1) / TF_FD_TILE : 0;
    const uint16_t* kbase = k_cache + (size_t)kv_h * HD;
    const uint16_t* vbase = v_cache + (size_t)kv_h * HD;
    uint8_t* ring = lds_raw + wave * TF_FD_WAVE;
    float* q_lds = reinterpret_cast<float*>(lds_raw + TF_FD_Q);

    // q: this wave copies heads 2 wave, 2 wave + 1 of the group (heads past
    // G repeat head G - 1 and are zeroed below)
    {
        const int h = min(2 * wave + (lane >> 5), G - 1);
        tf_lds_dma16(q + ((size_t)kv_h * G + h) * HD + 4 * (lane & 31),
                  tf_lds_off(q_lds) + wave * 1024);
    }
    // tile j -> slot b: four copies of 4 K rows (issue_k), four of 4 V rows
    // (issue_v); rows past the split repeat its last token (their scores
    // are masked)
    auto issue_k = [&](int j, int b) {
        const int t0 = t_begin + TF_FD_TILE * j;
        const uint32_t base = tf_lds_off(ring) + b * TF_FD_SLOT;
        const int r4 = lane >> 4;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 4 * i + r4;
            const int t = min(t0 + r, t_end - 1);
            tf_lds_dma16(kbase + (size_t)t * stride + 8 * (n ^ r), base + 1024 * i);
        }
    };
    auto issue_v = [&](int j, int b) {
        const int t0 = t_begin + TF_FD_TILE * j;
        const uint32_t base = tf_lds_off(ring) + b * TF_FD_SLOT;
        const int r4 = lane >> 4;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = min(t0 + 4 * i + r4, t_end - 1);
            tf_lds_dma16(vbase + (size_t)t * stride + 8 * n, base + 4096 + TF_FD_VBLK * i);
        }
    };
    // step of this wave: tiles j (slot 0) and j + 8 (slot 1), 32 tokens
    // under one softmax update.  Both K tiles are issued before both V
    // tiles: copies complete in issue order, so the scores and the softmax
    // run while the V rows are still arriving.
    auto issue_step = [&](int j) -> int {
        const bool two = j + TF_FD_WAVES < n_tiles;
        issue_k(j, 0);
        if (two) issue_k(j + TF_FD_WAVES, 1);
        issue_v(j, 0);
        if (two) issue_v(j + TF_FD_WAVES, 1);
        return two ? 2 : 1;
    };
    const int n_issued = wave < n_tiles ? issue_step(wave) : 0;
    // the q copy is older than the K/V copies: wait for it only
    if (n_issued == 2)
        asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if (n_issued == 1)
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    TF_FD_STAMP(1);
    __syncthreads();
    TF_FD_STAMP(2);

    // q fragments: head n, dims 32 g + 8 jj .. +7, as two f16 parts of
    // q 2^-e with e = ilogb(max |q|) - 14, so the group's largest element
    // lands in [2^14, 2^15) and the residual of every element is within
    // 2^-25 of the largest
    tf_h16x8 qa[4][2];
    {
        float qv[4][8];
        float qmax = 0.f;
        const bool hv = n < G;
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int h2 = 0; h2 < 2; h2++) {
                float4 v = *reinterpret_cast<const float4*>(q_lds + n * HD + 32 * g + 8 * jj + 4 * h2);
                if (!hv) v = make_float4(0.f, 0.f, 0.f, 0.f);
                qv[jj][4 * h2 + 0] = v.x;
                qv[jj][4 * h2 + 1] = v.y;
                qv[jj][4 * h2 + 2] = v.z;
                qv[jj][4 * h2 + 3] = v.w;
                qmax = fmaxf(qmax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
        qmax = tf_wave_max(qmax);
        const int e = qmax > 0.f ? ilogbf(qmax) - 14 : 0;
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x = ldexpf(qv[jj][i], -e);
                const _Float16 p0 = (_Float16)x;
                qa[jj][0][i] = p0;
                qa[jj][1][i] = (_Float16)(x - (float)p0);
            }
        scale = ldexpf(scale, e);
    }
    TF_FD_STAMP(3);

    float m = TF_NEG_BIG, l = 0.f;  // head n: running max, this lane's share of the sum
    tf_f32x4m o[8];                 // O^T of dims 16 db + 4 g + r, head n
#pragma unroll
    for (int db = 0; db < 8; db++) o[db] = tf_f32x4m{0.f, 0.f, 0.f, 0.f};
    // per-lane LDS byte offsets inside a slot
    uint32_t koff[4];
#pragma unroll
    for (int jj = 0; jj < 4; jj++) koff[jj] = n * 256 + 16 * ((4 * g + jj) ^ n);
    const uint32_t voff = 4096 + g * TF_FD_VBLK + 2 * n;

    // scores of tokens t0 + 4 g + r (r < 4), head n, from the K rows of a slot
    auto scores = [&](const uint8_t* slot, int t0, float (&sv)[4]) {
        tf_h16x8 kf[4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) kf[jj] = *reinterpret_cast<const tf_h16x8*>(slot + koff[jj]);
        tf_f32x4m c0 = tf_f32x4m{0.f, 0.f, 0.f, 0.f}, c1 = c0;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            c0 = tf_mfma_f16_k32(kf[jj], qa[jj][0], c0);
            c1 = tf_mfma_f16_k32(kf[jj], qa[jj][1], c1);
        }
        const tf_f32x4m c = c0 + c1;
#pragma unroll
        for (int r = 0; r < 4; r++) sv[r] = t0 + 4 * g + r < t_end ? c[r] * scale : TF_NEG_BIG;
    };
    // O^T += V^T P^T for one slot, hi and lo parts of p in one k = 32 step
    auto pv = [&](const uint8_t* slot, const tf_h16x8& pb) {
        _Float16 vv[8][4];
        const uint8_t* vp = slot + voff;
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                vv[db][i] = *reinterpret_cast<const _Float16*>(vp + 256 * i + 32 * db);
#pragma unroll
        for (int db = 0; db < 8; db++) {
            tf_h16x8 va;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                va[i] = vv[db][i];
                va[4 + i] = vv[db][i];
            }
            o[db] = tf_mfma_f16_k32(va, pb, o[db]);
        }
    };

    for (int j = wave; j < n_tiles; j += 2 * TF_FD_WAVES) {
        const bool two = j + TF_FD_WAVES < n_tiles;
        // the step's K tiles (the V copies, 4 per tile, may still be in flight)
        if (two)
            asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
#ifdef TF_FLASH_STAMPS
        if (j == wave) TF_FD_STAMP(4);
#endif
        const int t0 = t_begin + TF_FD_TILE * j;
        float sv[2][4];
        scores(ring, t0, sv[0]);
        if (two) {
            scores(ring + TF_FD_SLOT, t0 + TF_FD_TILE * TF_FD_WAVES, sv[1]);
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) sv[1][r] = TF_NEG_BIG;
        }
        // ---- online softmax of head n over the step's 32 tokens
        float tm = fmaxf(fmaxf(fmaxf(sv[0][0], sv[0][1]), fmaxf(sv[0][2], sv[0][3])),
                         fmaxf(fmaxf(sv[1][0], sv[1][1]), fmaxf(sv[1][2], sv[1][3])));
        tm = fmaxf(tm, __shfl_xor(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        const float m_new = fmaxf(m, tm);
        const float alpha = __expf(m - m_new);
        m = m_new;
        tf_h16x8 pb[2];
        float ps = 0.f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = sv[u][r] > 0.5f * TF_NEG_BIG ? __expf(sv[u][r] - m_new) : 0.f;
                ps += p;
                const _Float16 h0 = (_Float16)p;
                pb[u][r] = h0;
                pb[u][4 + r] = (_Float16)(p - (float)h0);
            }
        l = l * alpha + ps;
#pragma unroll
        for (int db = 0; db < 8; db++) o[db] *= alpha;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the V tiles
        pv(ring, pb[0]);
        if (two) pv(ring + TF_FD_SLOT, pb[1]);
        // both slots are consumed: refill them with the next step
        if (j + 2 * TF_FD_WAVES < n_tiles) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue_step(j + 2 * TF_FD_WAVES);
        }
    }
    TF_FD_STAMP(5);

    // ---- combine the eight waves: (m, l, O) of each through LDS
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    __syncthreads();  // every wave is done with its ring
    float* cmb = reinterpret_cast<float*>(lds_raw);  // [waves][16 heads][TF_FD_CR]
    float* row = cmb + (wave * 16 + n) * TF_FD_CR;
    if (g == 0) {
        row[0] = m;
        row[1] = l;
    }
#pragma unroll
    for (int db = 0; db < 8; db++)
        *reinterpret_cast<tf_f32x4m*>(row + 4 + 16 * db + 4 * g) = o[db];
    __syncthreads();
    TF_FD_STAMP(6);
    const int po = 2 + HD;
    for (int i = tid; i < G * HD; i += 64 * TF_FD_WAVES) {
        const int h = i >> 7, d = i & (HD - 1);
        float mw[TF_FD_WAVES], M = TF_NEG_BIG;
#pragma unroll
        for (int w = 0; w < TF_FD_WAVES; w++) {
            mw[w] = cmb[(w * 16 + h) * TF_FD_CR];
            M = fmaxf(M, mw[w]);
        }
        float O = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < TF_FD_WAVES; w++) {
            const float a = __expf(mw[w] - M);
            O += a * cmb[(w * 16 + h) * TF_FD_CR + 4 + d];
            L += a * cmb[(w * 16 + h) * TF_FD_CR + 1];
        }
        if (out) {  // workgroup-uniform; G * HD is a multiple of 64
            const float v = O / fmaxf(L, 1e-20f);
            const size_t oi = (size_t)kv_h * G * HD + i;
            out[oi] = v;
            if (q8) {  // this 32-lane half holds one 32-value group
                const float amax = tf_group32_max(fabsf(v));
                const float dq = amax * (1.0f / 127.0f);
                q8[oi] = (int8_t)tf_q8_value(v, amax, dq);
                if ((lane & 31) == 0) d8[oi >> 5] = dq;
            }
            continue;
        }
        float* base = partial + ((size_t)(kv_h * G + h) * n_split + s) * po;
        if (d == 0) {
            base[0] = M;
            base[1] = L;
        }
        base[2 + d] = O;
    }
#ifdef TF_FLASH_STAMPS
    TF_FD_STAMP(7);
    const int wg = blockIdx.y * gridDim.x + blockIdx.x;
    if (lane == 0 && wg < 4096 / TF_FD_WAVES)
#pragma unroll
        for (int k = 0; k < 8; k++) tf_fd_stamps[(size_t)(TF_FD_WAVES * wg + wave) * 8 + k] = st_[k];
#endif
}

// Log-sum-exp merge of the partitions (flash.cu:222-255).  Workgroup
// (head h, dim chunk c) produces dims 32c .. 32c+31 of head h; thread
// (sub, d) owns partitions sub, sub + 8, ... of dim d.  With n_split <= 128
// every (m, l, O) value a thread needs is loaded in one round before any of
// them is used (the merge is a chain of latencies, not of bytes): the
// workgroup maximum M goes through LDS, then each thread sums
// e^(m_s - M) O_s and e^(m_s - M) l_s over its partitions in order and the
// eight subset sums are added in order.  Longer split lists take the same
// steps in two passes over the partials.  With q8, the chunk's 32 outputs
// are one Q8 group.
template <int KMAX>  // partitions per thread held in registers (n_split <= 8 KMAX)
__device__ __forceinline__ void tf_flash_reduce_regs(const float* ph, int po, int d, int head_dim,
                                                     int n_split, int sub, float* red,
                                                     float& acc, float& lsum) {
    float mv[KMAX], lv[KMAX], ov[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
        const int s = sub + 8 * k;
        const bool live = s < n_split;
        const float* p = ph + (size_t)(live ? s : 0) * po;
        mv[k] = live ? p[0] : TF_NEG_BIG;
        lv[k] = live ? p[1] : 0.f;
        ov[k] = live && d < head_dim ? p[2 + d] : 0.f;
    }
    float mx = mv[0];
#pragma unroll
    for (int k = 1; k < KMAX; k++) mx = fmaxf(mx, mv[k]);
    if ((threadIdx.x & 31) == 0) red[sub] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int i = 1; i < 8; i++) M = fmaxf(M, red[i]);
    acc = 0.f;
    lsum = 0.f;
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
        const float a = sub + 8 * k < n_split ? __expf(mv[k] - M) : 0.f;
        acc += a * ov[k];
        lsum += a * lv[k];
    }
}

__global__ __launch_bounds__(256) void tf_flash_reduce_kernel(const float* __restrict__ partial,
                                                              float* __restrict__ out,
                                                              int8_t* __restrict__ q8,
                                                              float* __restrict__ d8,
                                                              int head_dim, int n_split) {
    __shared__ float red[256];
    __shared__ float lred[8];
    __shared__ float mred[8];
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const int po = 2 + head_dim;
    const float* ph = partial + (size_t)h * n_split * po;
    const int dl = tid & 31, sub = tid >> 5;
    const int d = 32 * blockIdx.y + dl;
    float acc, lsum;
    if (n_split <= 64) {
        tf_flash_reduce_regs<8>(ph, po, d, head_dim, n_split, sub, mred, acc, lsum);
    } else if (n_split <= 128) {
        tf_flash_reduce_regs<16>(ph, po, d, head_dim, n_split, sub, mred, acc, lsum);
    } else {
        float mx = TF_NEG_BIG;
        for (int s = sub; s < n_split; s += 8) mx = fmaxf(mx, ph[(size_t)s * po]);
        if (dl == 0) mred[sub] = mx;
        __syncthreads();
        float M = mred[0];
#pragma unroll
        for (int i = 1; i < 8; i++) M = fmaxf(M, mred[i]);
        acc = 0.f;
        lsum = 0.f;
#pragma unroll 8
        for (int s = sub; s < n_split; s += 8) {
            const float a = __expf(ph[(size_t)s * po] - M);
            acc += a * (d < head_dim ? ph[(size_t)s * po + 2 + d] : 0.f);
            lsum += a * ph[(size_t)s * po + 1];
        }
    }
    red[tid] = acc;
    if (dl == 0) lred[sub] = lsum;
    __syncthreads();
    if (tid < 32) {  // wave 0, lanes 0..31: the chunk's outputs
        float tot = 0.f, L = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            tot += red[32 * k + tid];
            L += lred[k];
        }
        const float v = d < head_dim ? tot / fmaxf(L, 1e-20f) : 0.f;
        const size_t i = (size_t)h * head_dim + d;
        if (d < head_dim) out[i] = v;
        if (q8) {  // quantize_q8 of the attention output: this 32-value group
            const float amax = tf_group32_max(fabsf(v));
            const float dq = amax * (1.0f / 127.0f);
            if (d < head_dim) {
                q8[i] = (int8_t)tf_q8_value(v, amax, dq);
                if (dl == 0) d8[i >> 5] = dq;
            }
        }
    }
}

// ---------------------------------------------------------------- dispatch

// The DMA kernel's LDS (138 KB) is above the default dynamic limit: raise
// it once per device.
static int tf_flash_dma_prepare() {
    static std::atomic<int> done[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
    if (done[dev].load(std::memory_order_acquire)) return 0;
    const hipError_t rc = hipFuncSetAttribute((const void*)tf_flash_partial_dma_kernel,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, TF_FD_LDS);
    if (rc != hipSuccess) return (int)rc;
    done[dev].store(1, std::memory_order_release);
    return 0;
}

template <int HD>
static int tf_flash_lds_bytes(int hpw) {
    const int gmax = 4 * hpw;
    return gmax * HD * 4 + gmax * TF_FLASH_TILE * 4 + TF_FLASH_TILE * (HD + 8) * 2 +
           TF_FLASH_TILE * HD * 2;
}

template <int HD>
static int tf_flash_launch_hd(const float* q, const uint16_t* k, const uint16_t* v,
                              float* partial, int n_head, int n_kv, int pos0,
                              const int* pos0_dev, int n_split, float scale,
                              tf_stream_t stream, float* out = nullptr, int8_t* q8 = nullptr,
                              float* d8 = nullptr) {
    const int G = n_head / n_kv;
    const dim3 grid(n_kv, n_split);
    if (HD == 128 && G <= 16) {  // the DMA-fed matrix-core partial
        const int rc = tf_flash_dma_prepare();
        if (rc) return rc;
        hipLaunchKernelGGL(tf_flash_partial_dma_kernel, grid, dim3(64 * TF_FD_WAVES), TF_FD_LDS,
                           tf_stream(stream), q, k, v, partial, n_head, n_kv, pos0, pos0_dev,
                           n_split, scale, out, q8, d8);
        return TF_LAUNCH_RESULT();
    }
    if (G <= 4)
        hipLaunchKernelGGL((tf_flash_partial_kernel<HD, 1>), grid, dim3(256),
                           tf_flash_lds_bytes<HD>(1), tf_stream(stream), q, k, v, partial, n_head,
                           n_kv, pos0, pos0_dev, n_split, scale);
    else if (G <= 8)
        hipLaunchKernelGGL((tf_flash_partial_kernel<HD, 2>), grid, dim3(256),
                           tf_flash_lds_bytes<HD>(2), tf_stream(stream), q, k, v, partial, n_head,
                           n_kv, pos0, pos0_dev, n_split, scale);
    else
        hipLaunchKernelGGL((tf_flash_partial_kernel<HD, 4>), grid, dim3(256),
                           tf_flash_lds_bytes<HD>(4), tf_stream(stream), q, k, v, partial, n_head,
                           n_kv, pos0, pos0_dev, n_split, scale);
    return TF_LAUNCH_RESULT();
}

static int tf_flash_partial_any(const float* q, const uint16_t* k, const uint16_t* v,
                                float* partial, int n_head, int n_kv, int head_dim, int pos0,
                                const int* pos0_dev, int n_q, int n_split, float scale,
                                tf_stream_t stream) {
    TF_CHECK_ARG(q && k && v && partial && n_head > 0 && n_kv > 0 && n_head % n_kv == 0);
    TF_CHECK_ARG(n_head / n_kv <= 16 && n_q == 1 && n_split >= 1 && n_split <= 1024);
    TF_CHECK_ARG(pos0_dev || pos0 >= 0);
    TF_CHECK_ARG(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0);
    switch (head_dim) {
    case 64:
        return tf_flash_launch_hd<64>(q, k, v, partial, n_head, n_kv, pos0, pos0_dev, n_split,
                                      scale, stream);
    case 128:
        return tf_flash_launch_hd<128>(q, k, v, partial, n_head, n_kv, pos0, pos0_dev, n_split,
                                       scale, stream);
    case 256:
        return tf_flash_launch_hd<256>(q, k, v, partial, n_head, n_kv, pos0, pos0_dev, n_split,
                                       scale, stream);
    default:
        return (int)hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------- C ABI

extern "C" int tf_flash_decode_partial(const float* q, const uint16_t* k_cache,
                                       const uint16_t* v_cache, float* partial, int n_head,
                                       int n_kv, int head_dim, int pos0, int n_q, int n_split,
                                       float scale, tf_stream_t stream) {
    return tf_flash_partial_any(q, k_cache, v_cache, partial, n_head, n_kv, head_dim, pos0,
                                nullptr, n_q, n_split, scale, stream);
}

extern "C" int tf_flash_decode_partial_d(const float* q, const uint16_t* k_cache,
                                         const uint16_t* v_cache, float* partial, int n_head,
                                         int n_kv, int head_dim, const int* pos0_dev, int n_q,
                                         int n_split, float scale, tf_stream_t stream) {
    TF_CHECK_ARG(pos0_dev != nullptr);
    return tf_flash_partial_any(q, k_cache, v_cache, partial, n_head, n_kv, head_dim, 0,
                                pos0_dev, n_q, n_split, scale, stream);
}

extern "C" int tf_flash_decode_reduce(const float* partial, float* out, int n_head,
                                      int head_dim, int n_split, int n_q, tf_stream_t stream) {
    TF_CHECK_ARG(partial && out && n_head > 0 && head_dim > 0 && n_split >= 1 && n_q == 1);
    TF_CHECK_ARG(head_dim <= 256 && n_split <= 1024);
    hipLaunchKernelGGL(tf_flash_reduce_kernel, dim3(n_head, (head_dim + 31) / 32), dim3(256), 0,
                       tf_stream(stream), partial, out, nullptr, nullptr, head_dim, n_split);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_flash_decode_reduce_q8(const float* partial, float* out, int8_t* q8, float* d8,
                                         int n_head, int head_dim, int n_split,
                                         tf_stream_t stream) {
    TF_CHECK_ARG(partial && out && q8 && d8 && n_head > 0 && n_split >= 1 && n_split <= 1024);
    TF_CHECK_ARG(head_dim > 0 && head_dim <= 256 && (head_dim % 64) == 0);
    hipLaunchKernelGGL(tf_flash_reduce_kernel, dim3(n_head, (head_dim + 31) / 32), dim3(256), 0,
                       tf_stream(stream),
                       partial, out, q8, d8, head_dim, n_split);
    return TF_LAUNCH_RESULT();
}

extern "C" int tf_flash_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                               float* partial, unsigned* counters, float* out, int8_t* q8,
                               float* d8, int n_head, int n_kv, int head_dim, int pos0,
                               const int* pos0_dev, int n_split, float scale,
                               tf_stream_t stream) {
    TF_CHECK_ARG(out && ((q8 == nullptr) == (d8 == nullptr)));
    (void)counters;  // reserved (may be NULL)
    TF_CHECK_ARG(n_kv > 0 && n_head > 0 && n_head % n_kv == 0);
    // One partition on the DMA-fed kernel: it writes the output itself.
    // Otherwise the merge runs as its own kernel.  Merging inside the partial
    // launch measured slower: with a release fence per workgroup (the last
    // one of a kv head merges) 14.2 vs 9.7 us at L = 512, 43.9 vs 10.8 us at
    // 4096; with 4 G merge workgroups per kv head polling a device-coherent
    // count of finished splits, 10.0 vs 8.3 us at 512 and 17.2 vs 15.1 us at
    // 32768; with a ticket per kv head (stores drained, the last split merges
    // with all its partial loads issued at once), 9.3 vs 8.1 us at 512 and
    // 15.2 vs 13.9 us at 4096 (8 splits).
    if (n_split == 1 && head_dim == 128 && n_head / n_kv <= 16) {
        TF_CHECK_ARG(q && k_cache && v_cache && (pos0_dev || pos0 >= 0));
        TF_CHECK_ARG(((uintptr_t)q & 15) == 0 && ((uintptr_t)k_cache & 15) == 0 &&
                     ((uintptr_t)v_cache & 15) == 0);
        return tf_flash_launch_hd<128>(q, k_cache, v_cache, partial, n_head, n_kv, pos0,
                                       pos0_dev, 1, scale, stream, out, q8, d8);
    }
    const int rc = tf_flash_partial_any(q, k_cache, v_cache, partial, n_head, n_kv, head_dim,
                                        pos0, pos0_dev, 1, n_split, scale, stream);
    if (rc) return rc;
    TF_CHECK_ARG(head_dim <= 256 && n_split <= 1024);
    hipLaunchKernelGGL(tf_flash_reduce_kernel, dim3(n_head, (head_dim + 31) / 32), dim3(256), 0,
                       tf_stream(stream),
                       partial, out, q8, d8, head_dim, n_split);
    return TF_LAUNCH_RESULT();
}

// Split choice: at least one 64-token span per split, at most one
// workgroup per CU (the DMA-fed kernel holds 138 KB of LDS, so a second
// workgroup per CU only queues behind the first).  Measured back to back
// (16/2 heads, partial + merge): L = 4096 -> 64 splits, 9.3 us (32: 9.8);
// L = 32768 -> 128 splits, 15.3 us (256: 28.8); L = 131072 -> 128 splits,
// 33.9 us (256: 43.7).
#ifndef TF_FLASH_SPLIT_TILES
#define TF_FLASH_SPLIT_TILES 1
#endif
#ifndef TF_FLASH_SPLIT_WPC
#define TF_FLASH_SPLIT_WPC 1
#endif

extern "C" int tf_flash_decode_n_split(int n_kv, int max_seq) {
    if (n_kv <= 0 || max_seq <= 0) return 8;
    const int cus = tf_device_cus();
    // at least TF_FLASH_SPLIT_TILES 64-token tiles per split; aim for
    // TF_FLASH_SPLIT_WPC workgroups per CU; multiples of 8 as in the
    // reference's fixed split.
    int by_len = max_seq / (TF_FLASH_SPLIT_TILES * TF_FLASH_TILE);
    int by_cus = (TF_FLASH_SPLIT_WPC * cus + n_kv - 1) / n_kv;
    int n = by_len < by_cus ? by_len : by_cus;
    n = (n / 8) * 8;
    if (n < 8) n = 8;
    if (n > 1024) n = 1024;
    return n;
}
