"""Oracle pins for the Q4_K x Q8 GEMV family (kernels/gemv.cu:71-191, 367-403,
469-490, 1877-1905, 2243-2263, 2346-2707).

Pins, none of which re-types the oracle's formula:
- agreement (fp64) with an independent numpy GGML dequantizer (tests/_util);
- per-position one-hot tests over all 256 values of a super-block, with
  distinct per-sub-block scales, so a wrong lane/word/nibble or scale index
  fails;
- the min term alone (q = 0): y = -dmin * m_g * d8_g * sum(q8_g);
- the reference's floor of K to whole super-blocks (K = 896);
- split-K / pair / dual / qkv / ffn consistency with the single GEMV.
"""
import numpy as np
import pytest

import oracle
from taraference_amd import synth
from _util import (assert_ffn_close, assert_gemv_close, gemv_q4k_ref, q4k_scales_mins,
                   q8_dequant)


def make(n_rows, n_cols, seed):
    rng = np.random.default_rng(seed)
    w, cb = synth.q4k_matrix(rng, n_rows, n_cols)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    return w, cb, x, q8, d8


def test_scale_pack_roundtrip():
    rng = np.random.default_rng(0)
    sc = rng.integers(0, 64, (500, 8))
    m = rng.integers(0, 64, (500, 8))
    sc2, m2 = q4k_scales_mins(synth.pack_q4k_scales(sc, m))
    assert np.array_equal(sc, sc2) and np.array_equal(m, m2)


@pytest.mark.parametrize("n_rows,n_cols", [(256, 64), (2048, 96), (896, 128), (11008, 16)])
def test_q4k_vs_numpy_dequant(n_rows, n_cols):
    w, cb, x, q8, d8 = make(n_rows, n_cols, n_rows + n_cols)
    y64, absn = oracle.gemv_q4k_q8_f64(w, q8, d8, n_rows, n_cols, cb)
    ref = gemv_q4k_ref(w, n_rows, q8_dequant(q8, d8))
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12 * absn.max())
    y32 = oracle.gemv_q4k_q8(w, q8, d8, n_rows, n_cols, cb)
    assert_gemv_close(y32, ref, absn, "oracle fp32 (reference lane order)")


def one_block(d=1.0, dmin=0.0, sc=None, m=None, qs=None):
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    sc = np.arange(1, 9) if sc is None else sc
    m = np.zeros(8, int) if m is None else m
    blk[4:16] = synth.pack_q4k_scales(np.array([sc]), np.array([m]))[0]
    if qs is not None:
        blk[16:] = qs
    return blk


def test_q4k_every_position():
    """One-hot nibble at value p, one-hot q8 at p: y = sc[p//32] * 15 * d8."""
    sc = np.array([3, 5, 7, 11, 13, 17, 19, 23])
    for p in range(256):
        j, r = divmod(p, 64)
        qs = np.zeros(128, np.uint8)
        if r < 32:
            qs[32 * j + r] = 0x0F
        else:
            qs[32 * j + r - 32] = 0xF0
        blk = one_block(sc=sc, qs=qs)
        q8 = np.zeros(256, np.int8)
        q8[p] = 127
        d8 = np.full(8, 0.5, np.float32)
        dots, sums = oracle.q4k_block_dots(blk, q8, 1)
        exp = np.zeros(8, np.int32)
        exp[p // 32] = 15 * 127
        assert np.array_equal(dots, exp), p
        y = oracle.gemv_q4k_q8(blk, q8, d8, 256, 1, 144)
        assert y[0] == np.float32(sc[p // 32] * 15 * 127 * 0.5), p


def test_q4k_min_term():
    m = np.array([1, 9, 17, 25, 33, 41, 49, 63])
    blk = one_block(d=0.25, dmin=0.125, sc=np.zeros(8, int), m=m)
    rng = np.random.default_rng(5)
    q8 = rng.integers(-127, 128, 256).astype(np.int8)
    d8 = np.array([2.0 ** -k for k in range(8)], np.float32)
    dots, sums = oracle.q4k_block_dots(blk, q8, 1)
    assert np.all(dots == 0)
    assert np.array_equal(sums, q8.reshape(8, 32).astype(np.int32).sum(1))
    y64, _ = oracle.gemv_q4k_q8_f64(blk, q8, d8, 256, 1, 144)
    exp = -0.125 * np.sum(m * d8.astype(np.float64) * sums)
    assert y64[0] == exp


def test_q4k_extremes_int_range():
    qs = np.full(128, 0xFF, np.uint8)
    blk = one_block(sc=np.full(8, 63), m=np.full(8, 63), qs=qs)
    q8 = np.full(256, -127, np.int8)
    dots, sums = oracle.q4k_block_dots(blk, q8, 1)
    assert np.all(dots == 15 * -127 * 32) and np.all(sums == -127 * 32)


def test_q4k_k896_floor_semantics():
    """The reference reads floor(896/256) = 3 super-blocks (gemv.cu:484)."""
    w, cb, x, q8, d8 = make(896, 64, 7)
    assert cb == 576
    y = oracle.gemv_q4k_q8(w, q8, d8, 896, 64, cb)
    w2 = w.copy()
    w2[:, 3 * 144:] ^= 0x5A  # scramble the 4th stored super-block
    y2 = oracle.gemv_q4k_q8(w2, q8, d8, 896, 64, cb)
    assert np.array_equal(y, y2)
    xs = q8_dequant(q8, d8).copy()
    ref = gemv_q4k_ref(w, 768, xs)  # only the first 768 inputs count
    _, absn = oracle.gemv_q4k_q8_f64(w, q8, d8, 896, 64, cb)
    assert_gemv_close(y, ref, absn, "K=896")


def test_q4k_splitk_and_reduce():
    n_rows, n_cols = 11008, 48
    w, cb, x, q8, d8 = make(n_rows, n_cols, 11)
    y64, absn = oracle.gemv_q4k_q8_f64(w, q8, d8, n_rows, n_cols, cb)
    part = oracle.gemv_q4k_q8_splitk(w, q8, d8, n_rows, n_cols, cb, 4)
    res = np.random.default_rng(1).standard_normal(n_cols).astype(np.float32)
    bias = np.random.default_rng(2).standard_normal(n_cols).astype(np.float32)
    y = oracle.gemv_splitk_reduce(part, n_cols, 4, bias=bias, use_res=2, out=res)
    assert_gemv_close(y, y64 + res + bias, absn + np.abs(res) + np.abs(bias), "splitk")
    y1 = oracle.gemv_splitk_reduce(part, n_cols, 4, use_res=1, residual=res)
    assert_gemv_close(y1, y64 + res, absn + np.abs(res), "splitk res=1")


def test_q4k_pair_dual_qkv_ffn():
    n_rows = 2048
    rng = np.random.default_rng(3)
    wq, cb = synth.q4k_matrix(rng, n_rows, 64)
    wk, _ = synth.q4k_matrix(rng, n_rows, 16)
    wv, _ = synth.q4k_matrix(rng, n_rows, 16)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    bq = rng.standard_normal(64).astype(np.float32)
    bk = rng.standard_normal(16).astype(np.float32)
    bv = rng.standard_normal(16).astype(np.float32)
    tq, aq = oracle.gemv_q4k_q8_f64(wq, q8, d8, n_rows, 64, cb)
    tk, ak = oracle.gemv_q4k_q8_f64(wk, q8, d8, n_rows, 16, cb)
    tv, av = oracle.gemv_q4k_q8_f64(wv, q8, d8, n_rows, 16, cb)
    a, b = oracle.gemv_q4k_pair(wq, wk, q8, d8, n_rows, 64, 16, cb, bq, bk)
    assert_gemv_close(a, tq + bq, aq + abs(bq), "pair a")
    assert_gemv_close(b, tk + bk, ak + abs(bk), "pair b")
    q, k, v = oracle.gemv_q4k_qkv(wq, wk, wv, q8, d8, n_rows, 64, 16, 16, cb, bq, bk, bv)
    assert np.array_equal(q, oracle.gemv_q4k_q8(wq, q8, d8, n_rows, 64, cb, bias=bq))
    assert_gemv_close(v, tv + bv, av + abs(bv), "qkv v")
    g, u = oracle.gemv_q4k_dual(wq, wq[::-1].copy(), q8, d8, n_rows, 64, cb)
    tu, au = oracle.gemv_q4k_q8_f64(wq[::-1].copy(), q8, d8, n_rows, 64, cb)
    assert_gemv_close(g, tq, aq, "dual a")
    assert_gemv_close(u, tu, au, "dual b")
    for ways in (1, 2, 4, 8):
        h = oracle.gemv_q4k_ffn(wq, wq[::-1].copy(), q8, d8, n_rows, 64, cb, ways)
        assert_ffn_close(h, tq, aq, tu, au, f"ffn {ways}-way")
