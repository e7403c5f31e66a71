"""GPU parity of the Q8_0 / Q5_0 GEMVs (kernels/gemv.cu:1558-1841, 2117-2200,
2268-2343, 2710-2818) against the CPU oracle, through the C ABI.

The Q8 activation the GPU quantizes inside the GEMV is checked by its effect:
its Q8 bytes equal tf_quantize_q8's, so the int32 block sums equal the
oracle's and the outputs sit within the fp32 GEMV tolerance (1e-5 relative,
tests/_util.gemv_tol) of the fp64 truth of the oracle's Q8 activation.
Shapes: Qwen2.5-0.5B (K = 896: attn 896 -> 896/128, ffn 896 -> 4864, the
tied Q8_0 lm_head 896 -> 151936), the pair layout and the any-layout path
(odd block count, 2-byte aligned columns), ragged column counts, every
residual mode and the split-K partials, including empty splits.
"""
import numpy as np
import pytest

import oracle
from taraference_amd import capi, synth
from _gpu import P, S, call, dev, empty, host
from _util import assert_gemv_close

pytestmark = pytest.mark.gpu


def mat(fmt, rng, n_rows, n_cols, pad=0):
    w, cb = (synth.q8_0_matrix if fmt == "q8_0" else synth.q5_0_matrix)(rng, n_rows, n_cols)
    if pad:  # column stride with `pad` extra bytes (2-byte aligned columns)
        w = np.ascontiguousarray(np.pad(w, ((0, 0), (0, pad)), constant_values=0xA5))
        cb += pad
    return w, cb


def gpu_q8(x):
    xq, xd = empty(x.size, __import__("torch").int8), empty(x.size // 32)
    call("tf_quantize_q8", P(dev(x)), P(xq), P(xd), x.size, S())
    return xq, xd


@pytest.mark.parametrize("n_rows,n_cols,pad,use_res,bias", [
    (896, 4864, 0, 0, False),    # pair layout, ffn width
    (896, 896, 0, 2, True),      # in-place residual
    (896, 151936, 0, 0, False),  # tied Q8_0 lm_head of Qwen2.5-0.5B
    (2048, 300, 0, 1, True),     # 64 blocks: two pairs per quad
    (4864, 64, 0, 0, False),     # 152 blocks: more pairs than one quad pass
    (800, 77, 0, 1, False),      # 25 blocks: any-layout path
    (896, 129, 2, 0, True),      # 2-byte aligned columns: any-layout path
    (32, 5, 0, 0, False),        # one block, ragged
])
def test_q8_0_q8(gpu, n_rows, n_cols, pad, use_res, bias):
    print(f"q8_0 q8 {n_rows}x{n_cols} pad={pad}", flush=True)
    rng = np.random.default_rng(n_rows * 7 + n_cols)
    w, cb = mat("q8_0", rng, n_rows, n_cols, pad)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    b = rng.standard_normal(n_cols).astype(np.float32)
    r = rng.standard_normal(n_cols).astype(np.float32)
    y64, absn = oracle.gemv_q8_0_q8_f64(w, q8, d8, n_rows, n_cols, cb)
    extra = (r if use_res else 0) + (b if bias else 0)
    extra_abs = (np.abs(r) if use_res else 0) + (np.abs(b) if bias else 0)
    wd, xq, xd = dev(w), *gpu_q8(x)
    out = dev(r.copy())
    call("tf_gemv_q8_0_q8", P(wd), P(xq), P(xd), P(out), n_rows, n_cols, cb, int(bias),
         P(dev(b)) if bias else None, use_res, P(dev(r)) if use_res == 1 else None, S())
    y = host(out)
    assert_gemv_close(y, y64 + extra, absn + extra_abs, "q8_0 q8")
    if n_cols <= 4864:
        yo = oracle.gemv_q8_0_q8(w, q8, d8, n_rows, n_cols, cb, bias=b if bias else None,
                                 use_res=use_res, residual=r, out=r.copy())
        assert_gemv_close(y, yo.astype(np.float64), absn + extra_abs, "q8_0 vs oracle fp32")
    # f32 activation quantized in LDS: same Q8 bytes, so the same tolerance
    out2 = dev(r.copy())
    call("tf_gemv_q8_0_f32", P(wd), P(dev(x)), P(out2), n_rows, n_cols, cb, int(bias),
         P(dev(b)) if bias else None, use_res, P(dev(r)) if use_res == 1 else None, S())
    assert_gemv_close(host(out2), y64 + extra, absn + extra_abs, "q8_0 f32")


@pytest.mark.parametrize("n_rows,n_cols,pad", [(896, 4864, 0), (800, 100, 0), (896, 33, 2),
                                               (4864, 64, 0)])
def test_q8_0_splitk(gpu, n_rows, n_cols, pad):
    print(f"q8_0 splitk {n_rows}x{n_cols} pad={pad}", flush=True)
    rng = np.random.default_rng(n_rows + 11 * n_cols)
    w, cb = mat("q8_0", rng, n_rows, n_cols, pad)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    nb = n_rows // 32
    wd, xd_f32 = dev(w), dev(x)
    xq, xd = gpu_q8(x)
    for ns in (1, 3, 8, min(64, nb + 3)):
        part = empty(ns * n_cols)
        call("tf_gemv_q8_0_q8_splitk", P(wd), P(xq), P(xd), P(part), n_rows, n_cols, cb, ns,
             S())
        ref = oracle.gemv_q8_0_q8_splitk(w, q8, d8, n_rows, n_cols, cb, ns).reshape(ns, -1)
        got = host(part).reshape(ns, -1)
        for s in range(ns):
            lo, hi = nb * s // ns, nb * (s + 1) // ns
            if lo == hi:
                assert np.all(got[s] == 0), (ns, s)
                continue
            xs = np.zeros_like(q8)
            xs[lo * 32:hi * 32] = q8[lo * 32:hi * 32]
            t, a = oracle.gemv_q8_0_q8_f64(w, xs, d8, n_rows, n_cols, cb)
            assert_gemv_close(got[s], t, a, f"q8 split {s}/{ns}")
            assert_gemv_close(got[s], ref[s].astype(np.float64), a, f"q8 split oracle {s}/{ns}")
        # the f32-activation split-K (fp32 products)
        part2 = empty(ns * n_cols)
        call("tf_gemv_q8_0_f32_splitk", P(wd), P(xd_f32), P(part2), n_rows, n_cols, cb, ns,
             S())
        got2 = host(part2).reshape(ns, -1)
        ref2 = oracle.gemv_q8_0_f32_splitk(w, x, n_rows, n_cols, cb, ns).reshape(ns, -1)
        for s in range(ns):
            lo, hi = nb * s // ns, nb * (s + 1) // ns
            xs = np.zeros_like(x)
            xs[lo * 32:hi * 32] = x[lo * 32:hi * 32]
            t, a = oracle.gemv_q8_0_f32_f64(w, xs, n_rows, n_cols, cb)
            if lo == hi:
                assert np.all(got2[s] == 0)
                continue
            assert_gemv_close(got2[s], t, a, f"q8 f32 split {s}/{ns}")
            assert_gemv_close(got2[s], ref2[s].astype(np.float64), a, "q8 f32 split oracle")


@pytest.mark.parametrize("n_rows,n_cols,pad,use_res,bias", [
    (896, 896, 0, 0, True), (896, 4864, 0, 2, False), (896, 128, 2, 1, True),
    (800, 65, 0, 0, False), (4864, 96, 0, 0, False), (32, 3, 0, 1, False)])
def test_q5_0(gpu, n_rows, n_cols, pad, use_res, bias):
    print(f"q5_0 {n_rows}x{n_cols} pad={pad}", flush=True)
    rng = np.random.default_rng(n_rows * 3 + n_cols)
    w, cb = mat("q5_0", rng, n_rows, n_cols, pad)
    x = synth.activation(rng, n_rows)
    b = rng.standard_normal(n_cols).astype(np.float32)
    r = rng.standard_normal(n_cols).astype(np.float32)
    y64, absn = oracle.gemv_q5_0_f32_f64(w, x, n_rows, n_cols, cb)
    extra = (r if use_res else 0) + (b if bias else 0)
    extra_abs = (np.abs(r) if use_res else 0) + (np.abs(b) if bias else 0)
    wd, xdv = dev(w), dev(x)
    out = dev(r.copy())
    call("tf_gemv_q5_0_f32", P(wd), P(xdv), P(out), n_rows, n_cols, cb, int(bias),
         P(dev(b)) if bias else None, use_res, P(dev(r)) if use_res == 1 else None, S())
    y = host(out)
    assert_gemv_close(y, y64 + extra, absn + extra_abs, "q5_0")
    yo = oracle.gemv_q5_0_f32(w, x, n_rows, n_cols, cb, bias=b if bias else None,
                              use_res=use_res, residual=r, out=r.copy())
    assert_gemv_close(y, yo.astype(np.float64), absn + extra_abs, "q5_0 vs oracle fp32")
    nb = n_rows // 32
    for ns in (2, 5):
        part = empty(ns * n_cols)
        call("tf_gemv_q5_0_f32_splitk", P(wd), P(xdv), P(part), n_rows, n_cols, cb, ns, S())
        got = host(part).reshape(ns, -1)
        ref = oracle.gemv_q5_0_f32_splitk(w, x, n_rows, n_cols, cb, ns).reshape(ns, -1)
        for s in range(ns):
            lo, hi = nb * s // ns, nb * (s + 1) // ns
            if lo == hi:
                assert np.all(got[s] == 0)
                continue
            xs = np.zeros_like(x)
            xs[lo * 32:hi * 32] = x[lo * 32:hi * 32]
            t, a = oracle.gemv_q5_0_f32_f64(w, xs, n_rows, n_cols, cb)
            assert_gemv_close(got[s], t, a, f"q5 split {s}/{ns}")
            assert_gemv_close(got[s], ref[s].astype(np.float64), a, "q5 split oracle")


@pytest.mark.parametrize("fmt", ["q5_0", "q8_0"])
@pytest.mark.parametrize("bias", [True, False])
def test_qkv_and_qk(gpu, fmt, bias):
    # Qwen2.5-0.5B attention: 14 heads x 64 -> 896, 2 KV heads -> 128
    n_rows, nq, nk = 896, 896, 128
    print(f"{fmt} qkv bias={bias}", flush=True)
    rng = np.random.default_rng(5 + bias)
    wq, cb = mat(fmt, rng, n_rows, nq)
    wk, _ = mat(fmt, rng, n_rows, nk)
    wv, _ = mat(fmt, rng, n_rows, nk)
    x = synth.activation(rng, n_rows)
    bs = [rng.standard_normal(n).astype(np.float32) for n in (nq, nk, nk)]
    q, k, v = empty(nq), empty(nk), empty(nk)
    bp = [P(dev(b)) if bias else None for b in bs]
    call(f"tf_gemv_{fmt}_qkv", P(dev(wq)), P(dev(wk)), P(dev(wv)), P(dev(x)), P(q), P(k), P(v),
         n_rows, nq, nk, nk, cb, int(bias), *bp, S())
    if fmt == "q8_0":
        q8, d8 = oracle.quantize_q8(x)
        truth = lambda wm, n: oracle.gemv_q8_0_q8_f64(wm, q8, d8, n_rows, n, cb)
    else:
        truth = lambda wm, n: oracle.gemv_q5_0_f32_f64(wm, x, n_rows, n, cb)
    for got, wm, b, n in ((q, wq, bs[0], nq), (k, wk, bs[1], nk), (v, wv, bs[2], nk)):
        t, a = truth(wm, n)
        assert_gemv_close(host(got), t + (b if bias else 0), a + (np.abs(b) if bias else 0),
                          f"{fmt} qkv")
    if fmt == "q5_0":  # the dual launch (Q+K, or gate+up with n_q = n_k)
        oa, ob = empty(nq), empty(nk)
        call("tf_gemv_q5_0_qk", P(dev(wq)), P(dev(wk)), P(dev(x)), P(oa), P(ob), n_rows, nq, nk,
             cb, int(bias), bp[0], bp[1], S())
        for got, wm, b, n in ((oa, wq, bs[0], nq), (ob, wk, bs[1], nk)):
            t, a = truth(wm, n)
            assert_gemv_close(host(got), t + (b if bias else 0),
                              a + (np.abs(b) if bias else 0), "q5_0 qk")


def test_argument_errors(gpu):
    lib = capi.load()
    rng = np.random.default_rng(0)
    w, cb = mat("q8_0", rng, 64, 4)
    wd, x = dev(w), dev(synth.activation(rng, 64))
    out = empty(4)
    bad = [
        ("tf_gemv_q8_0_f32", (P(wd), P(x), P(out), 48, 4, cb, 0, None, 0, None, S())),  # K%32
        ("tf_gemv_q8_0_f32", (P(wd), P(x), P(out), 64, 4, 60, 0, None, 0, None, S())),  # cb
        ("tf_gemv_q5_0_f32", (P(wd), P(x), P(out), 32768, 4, 22 * 1024, 0, None, 0, None,
                              S())),  # f32 image beyond 64 KiB of LDS
        ("tf_gemv_q8_0_f32_splitk", (P(wd), P(x), P(out), 64, 4, cb, 0, S())),  # n_split
        ("tf_gemv_q8_0_f32", (P(wd), P(x), P(out), 64, 4, cb, 1, None, 0, None, S())),  # bias
    ]
    for name, args in bad:
        fn = getattr(lib, name)
        fn.argtypes = capi.SIGNATURES[name]
        assert fn(*args) != 0, name
