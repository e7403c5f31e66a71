"""Oracle pins for the Q8_0 / Q5_0 GEMVs (kernels/gemv.cu:1558-1635,
1725-1804, 2117-2200).

Pins: fp64 agreement with independent numpy dequantizers of the GGML Q8_0
and Q5_0 formats (tests/_util.py, vectorised, written from the format
definition); one-hot activations over every value position of a block,
built by an independent encoder (synth.q5_0_pack / q8_0_pack) from chosen
codes, so an index or bit-position slip (bit 16+t of qh read as 12+t, a
swapped nibble half) changes an exact output; brute-force int32 block sums;
a hand-computed block; split-K partials that sum to the full product, with
empty splits written as zero.
"""
import numpy as np
import pytest

import oracle
from taraference_amd import synth
from _util import assert_gemv_close, gemv_block32_ref, q8_dequant


def case(fmt, n_rows, n_cols, seed):
    rng = np.random.default_rng(seed)
    mk = synth.q8_0_matrix if fmt == "q8_0" else synth.q5_0_matrix
    w, cb = mk(rng, n_rows, n_cols)
    x = synth.activation(rng, n_rows)
    return w, cb, x


def test_hand_block():
    # one Q8_0 block d = 0.5, qs = 1..32; x = 1: y = 0.5 * 528
    w = synth.q8_0_pack(np.array([0.5]), np.arange(1, 33).reshape(1, 32))
    x = np.ones(32, np.float32)
    part = oracle.gemv_q8_0_f32_splitk(w, x, 32, 1, 34, 1)
    assert part[0] == 264.0
    q8, d8 = oracle.quantize_q8(x)
    assert oracle.gemv_q8_0_q8(w, q8, d8, 32, 1, 34)[0] == np.float32(0.5 * d8[0] * 127 * 528)
    # one Q5_0 block d = 2, codes 0..31 -> values 2 * (-16..15); x = 1: y = -32
    w5 = synth.q5_0_pack(np.array([2.0]), np.arange(32).reshape(1, 32))
    assert w5[0, 2:6].tolist() == [0, 0, 0xFF, 0xFF]  # codes 16..31 set bits 16..31
    assert oracle.gemv_q5_0_f32(w5, x, 32, 1, 22)[0] == -32.0


@pytest.mark.parametrize("fmt", ["q8_0", "q5_0"])
def test_one_hot_every_position(fmt):
    # 4 columns x 2 blocks of distinct codes and scales; e_i picks W[:, i]
    rng = np.random.default_rng(3)
    n_cols, nb = 4, 2
    d = np.array([0.25, 0.5, 1.0, 2.0, 4.0, 8.0, 0.125, 16.0])
    if fmt == "q8_0":
        q = rng.integers(-127, 128, (n_cols * nb, 32))
        w = synth.q8_0_pack(d, q).reshape(n_cols, -1)
        vals = d[:, None] * q
    else:
        q = rng.integers(0, 32, (n_cols * nb, 32))
        w = synth.q5_0_pack(d, q).reshape(n_cols, -1)
        vals = d[:, None] * (q - 16)
    vals = vals.reshape(n_cols, nb * 32)
    cb = w.shape[1]
    for i in range(nb * 32):
        x = np.zeros(nb * 32, np.float32)
        x[i] = 1.0
        if fmt == "q8_0":
            y = oracle.gemv_q8_0_f32_splitk(w, x, nb * 32, n_cols, cb, 1)
        else:
            y = oracle.gemv_q5_0_f32(w, x, nb * 32, n_cols, cb)
        assert np.array_equal(y, vals[:, i].astype(np.float32)), i
        y64, _ = (oracle.gemv_q8_0_f32_f64 if fmt == "q8_0" else oracle.gemv_q5_0_f32_f64)(
            w, x, nb * 32, n_cols, cb)
        assert np.array_equal(y64, vals[:, i]), i


@pytest.mark.parametrize("n_rows,n_cols", [(32, 9), (896, 64), (4864, 16), (800, 33)])
def test_q8_0_q8(n_rows, n_cols):
    w, cb, x = case("q8_0", n_rows, n_cols, n_rows + n_cols)
    q8, d8 = oracle.quantize_q8(x)
    nb = n_rows // 32
    sums = oracle.q8_0_block_sums(w, q8, n_rows, n_cols, cb)
    qs = w.reshape(n_cols, nb, 34)[:, :, 2:].copy().view(np.int8).astype(np.int64)
    assert np.array_equal(sums, (qs * q8.reshape(nb, 32).astype(np.int64)).sum(axis=2))
    ref = gemv_block32_ref(w, n_rows, q8_dequant(q8, d8), 34)
    y64, absn = oracle.gemv_q8_0_q8_f64(w, q8, d8, n_rows, n_cols, cb)
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12 * absn.max())
    r = np.random.default_rng(1).standard_normal(n_cols).astype(np.float32)
    b = np.random.default_rng(2).standard_normal(n_cols).astype(np.float32)
    y = oracle.gemv_q8_0_q8(w, q8, d8, n_rows, n_cols, cb, bias=b, use_res=1, residual=r)
    assert_gemv_close(y, ref + r + b, absn + np.abs(r) + np.abs(b), "q8_0 q8")
    for ns in (1, 3, 8, nb + 2):
        part = oracle.gemv_q8_0_q8_splitk(w, q8, d8, n_rows, n_cols, cb, ns).reshape(ns, -1)
        for s in range(ns):
            if nb * s // ns == nb * (s + 1) // ns:
                assert np.all(part[s] == 0)
        assert_gemv_close(part.sum(axis=0), ref, absn, f"q8_0 splitk {ns}")


@pytest.mark.parametrize("fmt", ["q8_0", "q5_0"])
@pytest.mark.parametrize("n_rows,n_cols", [(32, 9), (896, 64), (4864, 16), (800, 33)])
def test_f32_paths(fmt, n_rows, n_cols):
    bb = 34 if fmt == "q8_0" else 22
    w, cb, x = case(fmt, n_rows, n_cols, 7 * n_rows + n_cols)
    ref = gemv_block32_ref(w, n_rows, x, bb)
    f64 = oracle.gemv_q8_0_f32_f64 if fmt == "q8_0" else oracle.gemv_q5_0_f32_f64
    y64, absn = f64(w, x, n_rows, n_cols, cb)
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12 * absn.max())
    nb = n_rows // 32
    split = oracle.gemv_q8_0_f32_splitk if fmt == "q8_0" else oracle.gemv_q5_0_f32_splitk
    for ns in (1, 4, nb + 1):
        part = split(w, x, n_rows, n_cols, cb, ns).reshape(ns, -1)
        assert_gemv_close(part.sum(axis=0), ref, absn, f"{fmt} splitk {ns}")
        # each split is the product over its own block range
        for s in range(ns):
            lo, hi = nb * s // ns * 32, nb * (s + 1) // ns * 32
            xs = np.zeros_like(x)
            xs[lo:hi] = x[lo:hi]
            rs, ra = f64(w, xs, n_rows, n_cols, cb)
            assert_gemv_close(part[s], rs, ra, f"{fmt} split {s}/{ns}")
    if fmt == "q5_0":
        b = np.random.default_rng(4).standard_normal(n_cols).astype(np.float32)
        out0 = np.random.default_rng(5).standard_normal(n_cols).astype(np.float32)
        y = oracle.gemv_q5_0_f32(w, x, n_rows, n_cols, cb, bias=b, use_res=2, out=out0)
        assert_gemv_close(y, ref + out0 + b, absn + np.abs(out0) + np.abs(b), "q5_0")
