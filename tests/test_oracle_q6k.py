"""Oracle pins for the Q6_K GEMVs (kernels/gemv.cu:233-337, 405-438, 515-536,
1998-2115) and the compact repack (cuda/load.rs:145-159).

Pins: fp64 agreement with an independent numpy GGML Q6_K dequantizer (both
the Q8 path and the f32-activation path); one-hot tests over all 256 value
positions with distinct signed scales; extreme 6-bit values; byte identity of
the 210 -> 212 repack; k-way and split-K consistency.
"""
import numpy as np
import pytest

import oracle
from taraference_amd import synth
from _util import assert_gemv_close, gemv_q6k_ref, q8_dequant


def make(n_rows, n_cols, seed):
    rng = np.random.default_rng(seed)
    raw, cb = synth.q6k_matrix(rng, n_rows, n_cols)
    comp, ccb = synth.q6k_compact(raw, n_rows)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    return raw, cb, comp, ccb, x, q8, d8


def test_repack_byte_identity():
    raw, cb, comp, ccb, *_ = make(2048, 33, 1)
    o = oracle.q6k_compact_repack(raw, 2048, 33, cb)
    assert np.array_equal(o, comp)
    blocks = o.reshape(33, 8, 212)
    assert np.array_equal(blocks[:, :, :210], raw.reshape(33, 8, 210))
    assert np.all(blocks[:, :, 210:] == 0)


@pytest.mark.parametrize("n_rows,n_cols", [(256, 40), (2048, 64), (11008, 8)])
def test_q6k_q8_vs_numpy(n_rows, n_cols):
    raw, cb, comp, ccb, x, q8, d8 = make(n_rows, n_cols, n_rows + 3)
    ref = gemv_q6k_ref(raw, n_rows, q8_dequant(q8, d8))
    y64, absn = oracle.gemv_q6k_q8_f64(comp, 212, q8, d8, n_rows, n_cols, ccb)
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12 * absn.max())
    y64r, _ = oracle.gemv_q6k_q8_f64(raw, 210, q8, d8, n_rows, n_cols, cb)
    assert np.array_equal(y64, y64r)
    y = oracle.gemv_q6k_compact_q8(comp, q8, d8, n_rows, n_cols, ccb)
    assert_gemv_close(y, ref, absn, "q6 compact")
    for ways in (4, 8):
        yk = oracle.gemv_q6k_compact_q8_kway(comp, q8, d8, n_rows, n_cols, ccb, ways)
        assert_gemv_close(yk, ref, absn, f"q6 {ways}-way")
    part = oracle.gemv_q6k_compact_q8_splitk(comp, q8, d8, n_rows, n_cols, ccb, 4)
    ys = oracle.gemv_splitk_reduce(part, n_cols, 4)
    assert_gemv_close(ys, ref, absn, "q6 splitk")


@pytest.mark.parametrize("n_rows,n_cols", [(256, 40), (2048, 64)])
def test_q6k_f32_vs_numpy(n_rows, n_cols):
    raw, cb, comp, ccb, x, q8, d8 = make(n_rows, n_cols, n_rows + 5)
    ref = gemv_q6k_ref(raw, n_rows, x.astype(np.float64))
    y64, absn = oracle.gemv_q6k_f32_f64(raw, x, n_rows, n_cols, cb)
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12 * absn.max())
    bias = np.random.default_rng(0).standard_normal(n_cols).astype(np.float32)
    y = oracle.gemv_q6k_f32(raw, x, n_rows, n_cols, cb, bias=bias)
    assert_gemv_close(y, ref + bias, absn + np.abs(bias), "q6 f32")


def q6_block(vals, scales, d=1.0):
    """Build a 210-byte block from 6-bit values [256] (0..63) and int8 scales."""
    blk = np.zeros(210, np.uint8)
    v = np.asarray(vals).reshape(2, 4, 32)  # [half n, quarter k, l]
    ql = np.zeros((2, 64), np.uint8)
    qh = np.zeros((2, 32), np.uint8)
    ql[:, 0:32] = (v[:, 0] & 0xF) | ((v[:, 2] & 0xF) << 4)
    ql[:, 32:64] = (v[:, 1] & 0xF) | ((v[:, 3] & 0xF) << 4)
    qh[:] = (v[:, 0] >> 4) | ((v[:, 1] >> 4) << 2) | ((v[:, 2] >> 4) << 4) | ((v[:, 3] >> 4) << 6)
    blk[0:128] = ql.reshape(-1)
    blk[128:192] = qh.reshape(-1)
    blk[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    blk[208:210] = np.array([d], np.float16).view(np.uint8)
    return blk


def test_q6k_every_position():
    scales = np.array([3, -5, 7, -11, 13, -17, 19, -23, 29, -31, 2, -3, 5, -7, 11, -13])
    for p in range(256):
        vals = np.full(256, 32)  # weight 0 everywhere
        vals[p] = 63             # weight +31 at p
        blk = q6_block(vals, scales)
        comp = np.zeros(212, np.uint8)
        comp[:210] = blk
        q8 = np.zeros(256, np.int8)
        q8[p] = -127
        d8 = np.full(8, 0.25, np.float32)
        exp = np.zeros(16, np.int32)
        exp[p // 16] = 31 * -127
        assert np.array_equal(oracle.q6k_block_dots(blk, 210, q8, 1), exp), p
        assert np.array_equal(oracle.q6k_block_dots(comp, 212, q8, 1), exp), p
        y = oracle.gemv_q6k_compact_q8(comp, q8, d8, 256, 1, 212)
        assert y[0] == np.float32(scales[p // 16] * 31 * -127 * 0.25), p
        x = np.zeros(256, np.float32)
        x[p] = 0.5
        yf = oracle.gemv_q6k_f32(blk, x, 256, 1, 210)
        assert yf[0] == np.float32(scales[p // 16] * 31 * 0.5), p


def test_q6k_extremes():
    for v, w in ((0, -32), (63, 31)):
        blk = q6_block(np.full(256, v), np.full(16, -32))
        q8 = np.full(256, 127, np.int8)
        assert np.all(oracle.q6k_block_dots(blk, 210, q8, 1) == 16 * w * 127)
