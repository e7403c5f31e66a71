"""GPU parity of the fused decode kernels against compositions of the oracle's
unfused reference kernels, at the Qwen2.5-3B and -7B shapes.

The fused prologue (RMSNorm in the reference's summation order + Q8) is
bit-identical to the unfused kernels, so the Q8 bytes match exactly and the
outputs carry only the fp32 GEMV tolerance (tests/_util.gemv_tol);
K/V rows land in the f16 cache with the reference's round-half-up
conversion (compared within one f16 ulp plus that tolerance)."""
import numpy as np
import pytest
import torch

import oracle
from taraference_amd import synth
from _gpu import P, S, call, dev, empty, host
from _util import assert_ffn_close, assert_gemv_close

pytestmark = pytest.mark.gpu

SHAPES = {"3b": (2048, 16, 2, 128), "7b": (3584, 28, 4, 128), "tiny": (256, 2, 1, 128)}


@pytest.mark.parametrize("shape", ["3b", "7b", "tiny"])
@pytest.mark.parametrize("v_q6k", [True, False])
def test_fused_qkv_rope_kv(gpu, shape, v_q6k):
    e, nh, nkv, hd = SHAPES[shape]
    rng = np.random.default_rng(hash((shape, v_q6k)) & 0xFFFF)
    x = (rng.standard_normal(e) * 3).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, e).astype(np.float32)
    eps = 1e-6
    wq, cb = synth.q4k_matrix(rng, e, nh * hd)
    wk, _ = synth.q4k_matrix(rng, e, nkv * hd)
    wv, cbv = synth.q6k_matrix(rng, e, nkv * hd) if v_q6k else synth.q4k_matrix(rng, e, nkv * hd)
    bq = (rng.standard_normal(nh * hd) * 0.02).astype(np.float32)
    bk = (rng.standard_normal(nkv * hd) * 0.02).astype(np.float32)
    bv = (rng.standard_normal(nkv * hd) * 0.02).astype(np.float32)
    pos, seq, theta = 37, 64, 1e6
    stride = nkv * hd
    q = empty(nh * hd)
    kc = torch.zeros(seq * stride, dtype=torch.int16, device="cuda")
    vc = torch.zeros(seq * stride, dtype=torch.int16, device="cuda")
    call("tf_fused_norm_qkv_rope_kv", P(dev(x)), P(dev(nw)), eps, P(dev(wq)), P(dev(wk)),
         P(dev(wv)), 14 if v_q6k else 12, P(dev(bq)), P(dev(bk)), P(dev(bv)), e, nh, nkv, hd, cb,
         cbv, P(q), P(kc), P(vc), pos, None, theta, S())
    # oracle composition (layer.rs order)
    xb = oracle.rms_norm(x, nw, eps)
    q8, d8 = oracle.quantize_q8(xb)
    tq, aq = oracle.gemv_q4k_q8_f64(wq, q8, d8, e, nh * hd, cb)
    tk, ak = oracle.gemv_q4k_q8_f64(wk, q8, d8, e, nkv * hd, cb)
    if v_q6k:
        tv, av = oracle.gemv_q6k_f32_f64(wv, xb, e, nkv * hd, cbv)
    else:
        tv, av = oracle.gemv_q4k_q8_f64(wv, q8, d8, e, nkv * hd, cbv)
    tq, tk, tv = tq + bq, tk + bk, tv + bv

    def rope64(v, n_heads):
        out = v.copy().reshape(n_heads, hd)
        i = np.arange(hd // 2)
        freq = np.float32(theta) ** (-2.0 * i / hd)
        ang = pos * freq
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = out[:, : hd // 2].copy(), out[:, hd // 2:].copy()
        out[:, : hd // 2] = x0 * c - x1 * s
        out[:, hd // 2:] = x0 * s + x1 * c
        return out.reshape(-1)

    # A rotated output mixes the pair (x0, x1): its tolerance is the sum of
    # both inputs' GEMV tolerances (first order, |cos|, |sin| <= 1) plus
    # 1e-5 (|x0| + |x1|) for the fp32 angle and sincos.
    def rope_tol(v, a, n_heads):
        v, a = v.reshape(n_heads, hd), a.reshape(n_heads, hd)
        sv = np.maximum(np.abs(v), 0.1 * a)
        t = 1e-5 * (sv[:, : hd // 2] + sv[:, hd // 2:]) + 1e-5 * (
            np.abs(v[:, : hd // 2]) + np.abs(v[:, hd // 2:]))
        return np.concatenate([t, t], axis=1).reshape(-1)

    def check(got, ref, tol, what):
        err = np.abs(np.asarray(got, np.float64) - ref)
        assert np.all(err <= tol), (what, err.max(), int(np.argmax(err / tol)))

    check(host(q), rope64(tq, nh), rope_tol(tq, aq + np.abs(bq), nh), "q (rope)")
    K = host(kc).view(np.float16).reshape(seq, stride)[pos].astype(np.float64)
    V = host(vc).view(np.float16).reshape(seq, stride)[pos].astype(np.float64)
    rk = rope64(tk, nkv)
    ulpk = np.abs(np.spacing(rk.astype(np.float16))).astype(np.float64)
    check(K, rk, ulpk + rope_tol(tk, ak + np.abs(bk), nkv), "k (rope, f16)")
    ulpv = np.abs(np.spacing(tv.astype(np.float16))).astype(np.float64)
    check(V, tv, ulpv + 1e-5 * np.maximum(np.abs(tv), 0.1 * (av + np.abs(bv))), "v (f16)")
    # other cache rows untouched
    assert np.all(host(kc).reshape(seq, stride)[np.arange(seq) != pos] == 0)


@pytest.mark.parametrize("n_rows,n_cols", [(2048, 11008), (3584, 18944), (256, 100)])
def test_fused_ffn_norm(gpu, n_rows, n_cols):
    rng = np.random.default_rng(n_cols)
    g, cb = synth.q4k_matrix(rng, n_rows, n_cols)
    u, _ = synth.q4k_matrix(rng, n_rows, n_cols)
    x = (rng.standard_normal(n_rows) * 5).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, n_rows).astype(np.float32)
    h = empty(n_cols)
    call("tf_gemv_q4k_ffn_norm", P(dev(g)), P(dev(u)), P(dev(x)), P(dev(nw)), 1e-6, P(h), n_rows,
         n_cols, cb, S())
    xb = oracle.rms_norm(x, nw, 1e-6)
    q8, d8 = oracle.quantize_q8(xb)
    tg, ag = oracle.gemv_q4k_q8_f64(g, q8, d8, n_rows, n_cols, cb)
    tu, au = oracle.gemv_q4k_q8_f64(u, q8, d8, n_rows, n_cols, cb)
    assert_ffn_close(host(h), tg, ag, tu, au, "ffn_norm")


@pytest.mark.parametrize("n_rows,n_cols", [(11008, 2048), (18944, 3584), (512, 256)])
def test_q6k_compact_f32_inplace(gpu, n_rows, n_cols):
    rng = np.random.default_rng(n_rows)
    raw, _ = synth.q6k_matrix(rng, n_rows, n_cols)
    comp, ccb = synth.q6k_compact(raw, n_rows)
    x = synth.activation(rng, n_rows)
    r = rng.standard_normal(n_cols).astype(np.float32)
    out = dev(r)
    call("tf_gemv_q6k_compact_f32", P(dev(comp)), P(dev(x)), P(out), n_rows, n_cols, ccb, 2, S())
    q8, d8 = oracle.quantize_q8(x)
    y64, absn = oracle.gemv_q6k_q8_f64(comp, 212, q8, d8, n_rows, n_cols, ccb)
    assert_gemv_close(host(out), y64 + r, absn + np.abs(r), "q6 f32 in place")


@pytest.mark.parametrize("n_rows,n_cols", [(2048, 151936), (3584, 152064), (256, 1000)])
def test_head_argmax(gpu, n_rows, n_cols):
    rng = np.random.default_rng(n_cols)
    raw, _ = synth.q6k_matrix(rng, n_rows, n_cols)
    comp, ccb = synth.q6k_compact(raw, n_rows)
    x = (rng.standard_normal(n_rows) * 4).astype(np.float32)
    nw = np.ones(n_rows, np.float32)
    logits = empty(n_cols)
    key = torch.zeros(1024, dtype=torch.int64, device="cuda")  # TF_ARGMAX_SLOTS
    idx = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    call("tf_gemv_q6k_head_argmax", P(dev(comp)), P(dev(x)), P(dev(nw)), 1e-6, P(logits), n_rows,
         n_cols, ccb, P(key), S())
    call("tf_argmax_key_finalize", P(key), P(idx), S())
    xb = oracle.rms_norm(x, nw, 1e-6)
    q8, d8 = oracle.quantize_q8(xb)
    y64, absn = oracle.gemv_q6k_q8_f64(comp, 212, q8, d8, n_rows, n_cols, ccb)
    lg = host(logits)
    assert_gemv_close(lg, y64, absn, "head logits")
    i = int(host(idx)[0])
    assert i == int(np.argmax(lg))             # argmax of the logits it wrote
    assert not host(key).any()                 # finalize resets every slot
    top2 = np.sort(y64)[-2:]
    if top2[1] - top2[0] > 1e-5 * absn.max():  # unambiguous in fp64 too
        assert i == int(np.argmax(y64))


@pytest.mark.parametrize("n", [256, 896, 2048, 3584, 5120, 8192])
def test_norm_quant_bit_exact(gpu, n):
    """RMSNorm in the reference's summation order + Q8: f32 output and Q8
    bytes/scales bit-identical to the oracle (ops.cu:4-34, gemv.cu:43-65)."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * rng.uniform(0.1, 30)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    xb, q8, d8 = empty(n), empty(n, torch.int8), empty(n // 32)
    call("tf_norm_quant", P(dev(x)), P(dev(w)), 1e-6, P(xb), P(q8), P(d8), n, S())
    rx = oracle.rms_norm(x, w, 1e-6)
    rq, rd = oracle.quantize_q8(rx)
    assert np.array_equal(host(xb).view(np.uint32), rx.view(np.uint32))
    assert np.array_equal(host(q8), rq)
    assert np.array_equal(host(d8).view(np.uint32), rd.view(np.uint32))


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_flash_reduce_q8(gpu, hd):
    n_head, n_kv, L = 8, 2, 700
    rng = np.random.default_rng(hd)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    K, V = synth.kv_cache(rng, L, n_kv, hd), synth.kv_cache(rng, L, n_kv, hd)
    part, out = empty(n_head * 8 * (2 + hd)), empty(n_head * hd)
    q8, d8 = empty(n_head * hd, torch.int8), empty(n_head * hd // 32)
    call("tf_flash_decode_partial", P(dev(q)), P(dev(K)), P(dev(V)), P(part), n_head, n_kv, hd,
         L - 1, 1, 8, 0.09, S())
    call("tf_flash_decode_reduce_q8", P(part), P(out), P(q8), P(d8), n_head, hd, 8, S())
    o = host(out)
    ref = oracle.attn_f64(q, K, V, n_head, n_kv, hd, L, 0.09)
    assert np.abs(o - ref).max() < 2e-3
    rq, rd = oracle.quantize_q8(o)  # Q8 of exactly the f32 it wrote
    assert np.array_equal(host(q8), rq)
    assert np.array_equal(host(d8).view(np.uint32), rd.view(np.uint32))


@pytest.mark.parametrize("shape", ["3b", "7b"])
def test_fused_qkv_q8_source_matches_norm_source(gpu, shape):
    """tf_fused_qkv_rope_kv on tf_norm_quant's output is bit-identical to the
    prologue-normalizing tf_fused_norm_qkv_rope_kv (same Q8, same f32)."""
    e, nh, nkv, hd = SHAPES[shape]
    rng = np.random.default_rng(len(shape))
    x = (rng.standard_normal(e) * 3).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, e).astype(np.float32)
    wq, cb = synth.q4k_matrix(rng, e, nh * hd)
    wk, _ = synth.q4k_matrix(rng, e, nkv * hd)
    wv, cbv = synth.q6k_matrix(rng, e, nkv * hd)
    b = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in (nh * hd, nkv * hd, nkv * hd)]
    seq, stride, pos = 16, nkv * hd, 5
    outs = []
    for fused_norm in (True, False):
        q = empty(nh * hd)
        kc = torch.zeros(seq * stride, dtype=torch.int16, device="cuda")
        vc = torch.zeros(seq * stride, dtype=torch.int16, device="cuda")
        if fused_norm:
            call("tf_fused_norm_qkv_rope_kv", P(dev(x)), P(dev(nw)), 1e-6, P(dev(wq)), P(dev(wk)),
                 P(dev(wv)), 14, P(dev(b[0])), P(dev(b[1])), P(dev(b[2])), e, nh, nkv, hd, cb,
                 cbv, P(q), P(kc), P(vc), pos, None, 1e6, S())
        else:
            xb, q8, d8 = empty(e), empty(e, torch.int8), empty(e // 32)
            call("tf_norm_quant", P(dev(x)), P(dev(nw)), 1e-6, P(xb), P(q8), P(d8), e, S())
            call("tf_fused_qkv_rope_kv", P(q8), P(d8), P(xb), P(dev(wq)), P(dev(wk)), P(dev(wv)),
                 14, P(dev(b[0])), P(dev(b[1])), P(dev(b[2])), e, nh, nkv, hd, cb, cbv, P(q),
                 P(kc), P(vc), pos, None, 1e6, S())
        outs.append((host(q).copy(), host(kc).copy(), host(vc).copy()))
    for a, c in zip(outs[0], outs[1]):
        assert np.array_equal(a.view(np.uint8), c.view(np.uint8))


def test_head_argmax_q8_source(gpu):
    n_rows, n_cols = 2048, 151936
    rng = np.random.default_rng(1)
    raw, _ = synth.q6k_matrix(rng, n_rows, n_cols)
    comp, ccb = synth.q6k_compact(raw, n_rows)
    x = synth.activation(rng, n_rows)
    q8, d8 = oracle.quantize_q8(x)
    logits = empty(n_cols)
    key = torch.zeros(1024, dtype=torch.int64, device="cuda")  # TF_ARGMAX_SLOTS
    idx = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    call("tf_gemv_q6k_q8_argmax", P(dev(comp)), P(dev(q8)), P(dev(d8)), P(logits), n_rows,
         n_cols, ccb, P(key), S())
    call("tf_argmax_key_finalize", P(key), P(idx), S())
    lg = host(logits)
    y64, absn = oracle.gemv_q6k_q8_f64(comp, 212, q8, d8, n_rows, n_cols, ccb)
    assert_gemv_close(lg, y64, absn, "head q8")
    assert int(host(idx)[0]) == int(np.argmax(lg))


@pytest.mark.parametrize("n_head,n_kv,L,n_split", [(16, 2, 700, 8), (28, 4, 300, 8),
                                                   (2, 1, 50, 8), (16, 2, 5, 1),
                                                   (16, 2, 4096, 32), (16, 2, 9000, 64)])
def test_gemv_q4k_flash_out(gpu, n_head, n_kv, L, n_split):
    """wo with the attention merge in its prologue (flash.cu:222 reduce +
    quantize_q8 + gemv_q4_k_global, residual in place): merged row within
    2e-3 of the oracle reduce and of fp64 attention, its Q8 bit-exact against
    quantizing that row, and the GEMV within the GEMV tolerance of the
    oracle on that Q8."""
    hd = 128
    rng = np.random.default_rng(L + n_head)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    K, V = synth.kv_cache(rng, L, n_kv, hd), synth.kv_cache(rng, L, n_kv, hd)
    scale = float(np.float32(1 / np.sqrt(hd)))
    part = empty(n_head * n_split * (2 + hd))
    call("tf_flash_decode_partial", P(dev(q)), P(dev(K)), P(dev(V)), P(part), n_head, n_kv, hd,
         L - 1, 1, n_split, scale, S())
    n_rows, n_cols = n_head * hd, 2048
    w, cb = synth.q4k_matrix(rng, n_rows, n_cols)
    res = rng.standard_normal(n_cols).astype(np.float32)
    y = dev(res.copy())
    ao, aq, ad = empty(n_rows), empty(n_rows, torch.int8), empty(n_rows // 32)
    call("tf_gemv_q4k_flash_out", P(dev(w)), P(part), n_head, hd, n_split, P(y), n_cols, cb, 2,
         P(ao), P(aq), P(ad), S())
    o = host(ao)
    ref = oracle.flash_reduce(host(part), n_head, hd, n_split)
    assert np.abs(o - ref).max() < 2e-3
    assert np.abs(o - oracle.attn_f64(q, K, V, n_head, n_kv, hd, L, scale)).max() < 2e-3
    rq, rd = oracle.quantize_q8(o)
    assert np.array_equal(host(aq), rq)
    assert np.array_equal(host(ad).view(np.uint32), rd.view(np.uint32))
    y64, absn = oracle.gemv_q4k_q8_f64(w, rq, rd, n_rows, n_cols, cb)
    assert_gemv_close(host(y) - res, y64, absn, "flash_out wo")
