"""GPU parity of the HIP GEMV family against the CPU oracle, through the C ABI.

Integer stages (Q8 bytes and scales, per-sub-block int32 dot sums) must be
bit-exact; fp32 outputs must be within 1e-5 relative of the fp64 truth with a
floor of 0.1 * sum|terms| for cancelling rows (tests/_util.gemv_tol), and
within the same bound of the oracle's reference-order fp32 result.
Shapes: BASELINE configs 0 (Q4_K 896 -> 4864), 1a (gate+up 2048 -> 2x11008),
1b (Q6_K 11008 -> 2048), 1c (QKV 2048 -> 2048+256+256), the Qwen2.5-3B
lm_head (Q6_K 2048 -> 151936) and the 7B widths (3584, 18944).
"""
import numpy as np
import pytest
import torch

import oracle
from taraference_amd import synth
from _gpu import P, S, call, dev, empty, host
from _util import assert_ffn_close, assert_gemv_close

pytestmark = pytest.mark.gpu


def gpu_q8(x):
    xq = empty(x.size, torch.int8)
    xd = empty(x.size // 32)
    call("tf_quantize_q8", P(dev(x)), P(xq), P(xd), x.size, S())
    return xq, xd


@pytest.mark.parametrize("n", [32, 896, 2048, 3584, 11008, 18944])
def test_q8_bit_exact(gpu, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * rng.uniform(0.01, 100, n)).astype(np.float32)
    x[:32] = 0.0
    if n >= 64:
        x[32:64] = np.arange(32, dtype=np.float32) - 15.5  # includes x/d ties near .5
    xq, xd = gpu_q8(x)
    q_ref, d_ref = oracle.quantize_q8(x)
    assert np.array_equal(host(xq), q_ref)
    assert np.array_equal(host(xd).view(np.uint32), d_ref.view(np.uint32))


def q4k_case(n_rows, n_cols, seed):
    rng = np.random.default_rng(seed)
    w, cb = synth.q4k_matrix(rng, n_rows, n_cols)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    return w, cb, x, q8, d8


@pytest.mark.parametrize("n_rows,n_cols", [(896, 4864), (2048, 2560), (3584, 512),
                                           (11008, 2048), (256, 7), (18944, 64)])
def test_q4k_block_dots_exact(gpu, n_rows, n_cols):
    w, cb, x, q8, d8 = q4k_case(n_rows, n_cols, 1)
    nb = n_rows // 256
    dots, sums = empty(n_cols * nb * 8, torch.int32), empty(n_cols * nb * 8, torch.int32)
    call("tf_q4k_block_dots", P(dev(w)), P(dev(q8)), P(dots), P(sums), n_rows, n_cols, cb, S())
    gd, gs = host(dots).reshape(n_cols, -1), host(sums).reshape(n_cols, -1)
    for j in list(range(0, n_cols, max(1, n_cols // 97))) + [n_cols - 1]:
        rd, rs = oracle.q4k_block_dots(np.ascontiguousarray(w[j]), q8, nb)
        assert np.array_equal(gd[j], rd), j
        assert np.array_equal(gs[j], rs), j


@pytest.mark.parametrize("n_rows,n_cols,use_res,bias", [
    (896, 4864, 0, False),    # config 0 (floor to 3 super-blocks)
    (2048, 2048, 2, False),   # wo, residual in place
    (2048, 2048, 1, True),
    (11008, 2048, 2, False),  # Q4_K ffn_down (full K in one wave)
    (3584, 3584, 0, True),    # 7B width
    (18944, 256, 2, True),
    (256, 5, 0, False),       # ragged: fewer rows than one wave pass
    (1280, 1001, 2, True),    # five super-blocks (8 slots per row), odd row count
    (512, 3000, 1, False),    # two super-blocks (4 slots per row)
])
def test_q4k_gemv(gpu, n_rows, n_cols, use_res, bias):
    w, cb, x, q8, d8 = q4k_case(n_rows, n_cols, n_rows + n_cols)
    rng = np.random.default_rng(9)
    b = rng.standard_normal(n_cols).astype(np.float32) if bias else None
    r = rng.standard_normal(n_cols).astype(np.float32)
    out = dev(r.copy())
    resid = dev(r)
    call("tf_gemv_q4k_q8", P(dev(w)), P(dev(q8)), P(dev(d8)), P(out), n_rows, n_cols, cb,
         int(bias), P(dev(b)) if bias else None, use_res, P(resid) if use_res == 1 else None, S())
    y = host(out)
    y64, absn = oracle.gemv_q4k_q8_f64(w, q8, d8, n_rows, n_cols, cb)
    extra = (r if use_res else 0) + (b if bias else 0)
    extra_abs = (np.abs(r) if use_res else 0) + (np.abs(b) if bias else 0)
    assert_gemv_close(y, y64 + extra, absn + extra_abs, "gpu q4k")
    yo = oracle.gemv_q4k_q8(w, q8, d8, n_rows, n_cols, cb, bias=b, use_res=use_res,
                            residual=r, out=r.copy())
    assert_gemv_close(y, yo.astype(np.float64), absn + extra_abs, "gpu vs oracle fp32")


@pytest.mark.parametrize("n_rows,n_cols", [(896, 4864), (2048, 2048), (1280, 77)])
def test_q4k_gemv_unaligned_activation(gpu, n_rows, n_cols):
    """Narrow rows (K <= 2048) read a 16-byte aligned Q8 activation straight
    from global memory; an activation one byte off that alignment is staged
    through LDS instead.  Both within the GEMV bound of the fp64 truth, and
    within a few fp32 roundings of each other."""
    w, cb, x, q8, d8 = q4k_case(n_rows, n_cols, 3 * n_rows + n_cols)
    wd = dev(w)
    buf = empty(n_rows + 64, torch.int8)
    buf[1:1 + n_rows].copy_(dev(q8))
    xd = dev(d8)
    outs = []
    for q in (dev(q8), buf[1:1 + n_rows]):
        o = empty(n_cols)
        call("tf_gemv_q4k_q8", P(wd), P(q), P(xd), P(o), n_rows, n_cols, cb, 0, None, 0, None,
             S())
        outs.append(host(o))
    y64, absn = oracle.gemv_q4k_q8_f64(w, q8, d8, n_rows, n_cols, cb)
    for y in outs:
        assert_gemv_close(y, y64, absn, "q4k gemv")
    assert np.abs(outs[0] - outs[1]).max() <= 1e-5 * absn.max()


def test_q4k_qkv_and_pair(gpu):
    n_rows = 2048
    rng = np.random.default_rng(13)
    wq, cb = synth.q4k_matrix(rng, n_rows, 2048)
    wk, _ = synth.q4k_matrix(rng, n_rows, 256)
    wv, _ = synth.q4k_matrix(rng, n_rows, 256)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    bq, bk, bv = (rng.standard_normal(n).astype(np.float32) for n in (2048, 256, 256))
    xq, xd = gpu_q8(x)
    q, k, v = empty(2048), empty(256), empty(256)
    call("tf_gemv_q4k_qkv", P(dev(wq)), P(dev(wk)), P(dev(wv)), P(xq), P(xd), P(q), P(k), P(v),
         n_rows, 2048, 256, 256, cb, 1, P(dev(bq)), P(dev(bk)), P(dev(bv)), S())
    for got, wm, b, n in ((q, wq, bq, 2048), (k, wk, bk, 256), (v, wv, bv, 256)):
        t, a = oracle.gemv_q4k_q8_f64(wm, q8, d8, n_rows, n, cb)
        assert_gemv_close(host(got), t + b, a + np.abs(b), "qkv")
    oa, ob = empty(2048), empty(256)
    call("tf_gemv_q4k_pair", P(dev(wq)), P(dev(wk)), P(xq), P(xd), P(oa), P(ob), n_rows,
         2048, 256, cb, 1, P(dev(bq)), P(dev(bk)), S())
    for got, wm, b, n in ((oa, wq, bq, 2048), (ob, wk, bk, 256)):
        t, a = oracle.gemv_q4k_q8_f64(wm, q8, d8, n_rows, n, cb)
        assert_gemv_close(host(got), t + b, a + np.abs(b), "pair")


@pytest.mark.parametrize("n_rows,n_cols", [(2048, 11008), (3584, 1000), (896, 300), (11008, 64)])
def test_q4k_ffn_dual(gpu, n_rows, n_cols):
    rng = np.random.default_rng(n_cols)
    g, cb = synth.q4k_matrix(rng, n_rows, n_cols)
    u, _ = synth.q4k_matrix(rng, n_rows, n_cols)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    tg, ag = oracle.gemv_q4k_q8_f64(g, q8, d8, n_rows, n_cols, cb)
    tu, au = oracle.gemv_q4k_q8_f64(u, q8, d8, n_rows, n_cols, cb)
    gd, ud = dev(g), dev(u)
    if n_rows % 256 == 0:
        h = empty(n_cols)
        call("tf_gemv_q4k_ffn_f32", P(gd), P(ud), P(dev(x)), P(h), n_rows, n_cols, cb, S())
        assert_ffn_close(host(h), tg, ag, tu, au, "ffn_f32")
    xq, xd = gpu_q8(x)
    h2 = empty(n_cols)
    call("tf_gemv_q4k_ffn", P(gd), P(ud), P(xq), P(xd), P(h2), n_rows, n_cols, cb, S())
    assert_ffn_close(host(h2), tg, ag, tu, au, "ffn")
    oa, ob = empty(n_cols), empty(n_cols)
    call("tf_gemv_q4k_dual", P(gd), P(ud), P(xq), P(xd), P(oa), P(ob), n_rows, n_cols, cb, S())
    assert_gemv_close(host(oa), tg, ag, "dual a")
    assert_gemv_close(host(ob), tu, au, "dual b")


@pytest.mark.parametrize("n_split", [1, 3, 4, 8])
def test_q4k_splitk_reduce(gpu, n_split):
    n_rows, n_cols = 11008, 2048
    w, cb, x, q8, d8 = q4k_case(n_rows, n_cols, 21)
    part = empty(n_split * n_cols)
    call("tf_gemv_q4k_q8_splitk", P(dev(w)), P(dev(q8)), P(dev(d8)), P(part), n_rows, n_cols,
         cb, n_split, S())
    pref = oracle.gemv_q4k_q8_splitk(w, q8, d8, n_rows, n_cols, cb, n_split)
    got = host(part)
    # each partial is itself a GEMV over a super-block range
    nb = n_rows // 256
    for s in range(n_split):
        b0, b1 = nb * s // n_split, nb * (s + 1) // n_split
        sub = np.ascontiguousarray(w[:, b0 * 144:b1 * 144])
        t, a = oracle.gemv_q4k_q8_f64(sub, np.ascontiguousarray(q8[b0 * 256:]),
                                      np.ascontiguousarray(d8[b0 * 8:]), (b1 - b0) * 256,
                                      n_cols, (b1 - b0) * 144)
        assert_gemv_close(got[s * n_cols:(s + 1) * n_cols], t, a, f"partial {s}")
    r = np.random.default_rng(2).standard_normal(n_cols).astype(np.float32)
    out = dev(r)
    call("tf_gemv_splitk_reduce", P(part), P(out), n_cols, n_split, 0, None, 2, None, S())
    y64, absn = oracle.gemv_q4k_q8_f64(w, q8, d8, n_rows, n_cols, cb)
    assert_gemv_close(host(out), y64 + r, absn + np.abs(r), "reduce")
    yo = oracle.gemv_splitk_reduce(pref, n_cols, n_split, use_res=2, out=r)
    assert_gemv_close(host(out), yo.astype(np.float64), absn + np.abs(r), "reduce vs oracle")


def q6_case(n_rows, n_cols, seed):
    rng = np.random.default_rng(seed)
    raw, cb = synth.q6k_matrix(rng, n_rows, n_cols)
    comp, ccb = synth.q6k_compact(raw, n_rows)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    return raw, cb, comp, ccb, x, q8, d8


@pytest.mark.parametrize("n_rows,n_cols", [(11008, 2048), (2048, 1000), (256, 3)])
def test_q6k_block_dots_exact(gpu, n_rows, n_cols):
    raw, cb, comp, ccb, x, q8, d8 = q6_case(n_rows, n_cols, 4)
    nb = n_rows // 256
    for blob, bb, colb in ((comp, 212, ccb), (raw, 210, cb)):
        dots = empty(n_cols * nb * 16, torch.int32)
        call("tf_q6k_block_dots", P(dev(blob)), bb, P(dev(q8)), P(dots), n_rows, n_cols, colb, S())
        gd = host(dots).reshape(n_cols, -1)
        for j in list(range(0, n_cols, max(1, n_cols // 61))) + [n_cols - 1]:
            rd = oracle.q6k_block_dots(np.ascontiguousarray(blob[j]), bb, q8, nb)
            assert np.array_equal(gd[j], rd), (bb, j)


@pytest.mark.parametrize("n_rows,n_cols,entry,use_res,bias", [
    (11008, 2048, "tf_gemv_q6k_down_splitk", 2, False),   # config 1b
    (18944, 512, "tf_gemv_q6k_down_splitk", 2, True),
    (2048, 151936, "tf_gemv_q6k_compact_q8", 0, False),   # Qwen2.5-3B lm_head
    # the LDS-fed wide kernel: K = 2048 with a ragged last four-row task, K = 1024
    (2048, 65539, "tf_gemv_q6k_compact_q8", 0, False),
    (1024, 70001, "tf_gemv_q6k_compact_q8", 0, False),
    (3584, 300, "tf_gemv_q6k_compact_q8", 1, True),
    (256, 9, "tf_gemv_q6k_compact_q8", 0, False),
])
def test_q6k_gemv(gpu, n_rows, n_cols, entry, use_res, bias):
    raw, cb, comp, ccb, x, q8, d8 = q6_case(n_rows, n_cols, n_cols)
    rng = np.random.default_rng(3)
    b = rng.standard_normal(n_cols).astype(np.float32) if bias else None
    r = rng.standard_normal(n_cols).astype(np.float32)
    out, resid = dev(r.copy()), dev(r)
    xq, xd = gpu_q8(x)
    call(entry, P(dev(comp)), P(xq), P(xd), P(out), n_rows, n_cols, ccb, int(bias),
         P(dev(b)) if bias else None, use_res, P(resid) if use_res == 1 else None, S())
    y64, absn = oracle.gemv_q6k_q8_f64(comp, 212, q8, d8, n_rows, n_cols, ccb)
    extra = (r if use_res else 0) + (b if bias else 0)
    extra_abs = (np.abs(r) if use_res else 0) + (np.abs(b) if bias else 0)
    assert_gemv_close(host(out), y64 + extra, absn + extra_abs, entry)


def test_q6k_splitk(gpu):
    n_rows, n_cols, n_split = 11008, 1024, 4
    raw, cb, comp, ccb, x, q8, d8 = q6_case(n_rows, n_cols, 8)
    part, out = empty(n_split * n_cols), empty(n_cols)
    call("tf_gemv_q6k_compact_q8_splitk", P(dev(comp)), P(dev(q8)), P(dev(d8)), P(part), n_rows,
         n_cols, ccb, n_split, S())
    call("tf_gemv_splitk_reduce", P(part), P(out), n_cols, n_split, 0, None, 0, None, S())
    y64, absn = oracle.gemv_q6k_q8_f64(comp, 212, q8, d8, n_rows, n_cols, ccb)
    assert_gemv_close(host(out), y64, absn, "q6 splitk")


@pytest.mark.parametrize("n_rows,n_cols,bias", [(2048, 256, True), (3584, 512, True),
                                                (768, 33, False)])
def test_q6k_f32(gpu, n_rows, n_cols, bias):
    raw, cb, comp, ccb, x, q8, d8 = q6_case(n_rows, n_cols, 5)
    b = np.random.default_rng(1).standard_normal(n_cols).astype(np.float32)
    out = empty(n_cols)
    call("tf_gemv_q6k_f32", P(dev(raw)), P(dev(x)), P(out), n_rows, n_cols, cb, int(bias),
         P(dev(b)) if bias else None, 0, None, S())
    y64, absn = oracle.gemv_q6k_f32_f64(raw, x, n_rows, n_cols, cb)
    assert_gemv_close(host(out), y64 + (b if bias else 0), absn + (np.abs(b) if bias else 0),
                      "q6 f32")


def test_q6k_repack(gpu):
    raw, cb, comp, ccb, *_ = q6_case(11008, 64, 2)
    dst = torch.full((comp.size,), 0xAB, dtype=torch.uint8, device="cuda")
    call("tf_q6k_compact_repack", P(dev(raw)), P(dst), 11008, 64, cb, S())
    assert np.array_equal(host(dst), comp.reshape(-1))
