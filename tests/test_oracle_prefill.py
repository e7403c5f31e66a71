"""Oracle pins for the prefill GEMMs (kernels/gemm.cu:6-121 with the
dequantizers common.cu:64-84,164-186) and prefill attention
(kernels/attn/fast_v2.cu:12-103).

Pins: fp64 agreement with the independent numpy GGML dequantizers
(tests/_util.py); one-hot activations that must return, exactly, the f32
dequantized weight d*sc*q - dmin*m (Q4_K) or d*sc*q (Q6_K) evaluated in numpy
float32 at every one of the 256 positions; token independence (a batch equals
its tokens one at a time, bit for bit); the n_tok = 1 case against the
separately pinned Q6_K x f32 GEMV.  Attention: every query against the
textbook fp64 softmax attention over its causal prefix (or_attn_f64, pinned
in test_oracle_flash.py), causality (cache rows past a query's position do not
change it), and a one-key prefix returning V_0.
"""
import numpy as np
import pytest

import oracle
from taraference_amd import synth
from _util import assert_gemv_close, f16, gemm_ref, q4k_scales_mins

rng0 = np.random.default_rng


def case(fmt, n_rows, n_cols, n_tok, seed):
    rng = rng0(seed)
    w, cb = (synth.q4k_matrix if fmt == "q4k" else synth.q6k_matrix)(rng, n_rows, n_cols)
    x = rng.standard_normal((n_tok, n_rows)).astype(np.float32)
    return w, cb, x


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("n_rows,n_cols,n_tok", [(256, 40, 3), (2048, 24, 9), (896, 16, 5)])
def test_gemm_vs_numpy(fmt, n_rows, n_cols, n_tok):
    w, cb, x = case(fmt, n_rows, n_cols, n_tok, n_rows + n_tok)
    fn = oracle.gemm_q4k if fmt == "q4k" else oracle.gemm_q6k
    y = fn(w, x, n_rows, n_cols, cb, n_tok)
    ref, absn = gemm_ref(fmt, w, n_rows, x)
    for t in range(n_tok):
        assert_gemv_close(y[t], ref[t], absn[t], f"{fmt} gemm t={t}")
        # token independence, bit for bit
        assert np.array_equal(fn(w, x[t:t + 1], n_rows, n_cols, cb, 1)[0], y[t])


def test_gemm_q6k_single_token_matches_gemv():
    w, cb, x = case("q6k", 2048, 64, 1, 3)
    y = oracle.gemm_q6k(w, x, 2048, 64, cb, 1)[0]
    g = oracle.gemv_q6k_f32(w, x[0], 2048, 64, cb)
    y64, absn = oracle.gemv_q6k_f32_f64(w, x[0], 2048, 64, cb)
    assert_gemv_close(y, y64, absn, "gemm t=1")
    assert_gemv_close(g, y64, absn, "gemv")


def f32_deq_q4k(blk):
    """numpy float32 restatement of d*sc*q - dmin*m per value (the order the
    reference's dequantizer rounds in)."""
    d = np.float32(f16(blk[0:2].reshape(1, 2))[0])
    dmin = np.float32(f16(blk[2:4].reshape(1, 2))[0])
    sc, m = q4k_scales_mins(blk[4:16].reshape(1, 12))
    qs = blk[16:144].astype(np.int64).reshape(4, 32)
    out = np.zeros(256, np.float32)
    for c in range(4):
        for h in range(2):
            s = 2 * c + h
            q = (qs[c] >> (4 * h)) & 15
            out[64 * c + 32 * h: 64 * c + 32 * h + 32] = \
                (d * np.float32(sc[0, s])) * q.astype(np.float32) - dmin * np.float32(m[0, s])
    return out


def f32_deq_q6k(blk):
    d = np.float32(f16(blk[208:210].reshape(1, 2))[0])
    sc = blk[192:208].view(np.int8).astype(np.float32)
    from _util import q6k_quants
    q = q6k_quants(blk.reshape(1, -1))[0].astype(np.float32)
    return (d * sc[np.arange(256) // 16]) * q


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
def test_gemm_one_hot_every_position(fmt):
    w, cb, _ = case(fmt, 256, 3, 1, 17)
    x = np.eye(256, dtype=np.float32)  # 256 tokens, token t = e_t
    fn = oracle.gemm_q4k if fmt == "q4k" else oracle.gemm_q6k
    y = fn(w, x, 256, 3, cb, 256)
    for j in range(3):
        blk = w[j, : (144 if fmt == "q4k" else 210)]
        ref = f32_deq_q4k(blk) if fmt == "q4k" else f32_deq_q6k(blk)
        assert np.array_equal(y[:, j], ref), j


def kv(rng, L, n_kv, hd):
    return synth.kv_cache(rng, L, n_kv, hd), synth.kv_cache(rng, L, n_kv, hd)


@pytest.mark.parametrize("n_head,n_kv,hd,pos0,n_q", [(4, 2, 64, 0, 7), (16, 2, 128, 40, 70),
                                                       (2, 1, 256, 3, 5), (14, 2, 64, 100, 3)])
def test_attn_prefill_vs_textbook(n_head, n_kv, hd, pos0, n_q):
    rng = rng0(n_q + pos0)
    L = pos0 + n_q
    K, V = kv(rng, L, n_kv, hd)
    q = rng.standard_normal((n_q, n_head * hd)).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(hd)))
    out = oracle.attn_prefill(q, K, V, n_head, n_kv, hd, pos0, n_q, scale)
    for qi in range(n_q):
        ref = oracle.attn_f64(q[qi], K, V, n_head, n_kv, hd, pos0 + qi + 1, scale)
        assert np.max(np.abs(out[qi] - ref)) < 1e-5, qi
    # causality: rows past the last position do not matter
    K2, V2 = K.copy(), V.copy()
    K2[pos0 + 1:] ^= 0x1234
    V2[pos0 + 1:] ^= 0x0F0F
    out2 = oracle.attn_prefill(q[:1], K2, V2, n_head, n_kv, hd, pos0, 1, scale)
    assert np.array_equal(out2[0], out[0])


def test_attn_prefill_first_query_is_v0():
    rng = rng0(9)
    K, V = kv(rng, 4, 1, 64)
    q = rng.standard_normal((2, 2 * 64)).astype(np.float32)
    out = oracle.attn_prefill(q, K, V, 2, 1, 64, 0, 2, 0.125)
    v0 = V[0].view(np.float16).astype(np.float32)
    assert np.array_equal(out[0, :64], v0) and np.array_equal(out[0, 64:], v0)
