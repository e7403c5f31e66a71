"""GPU parity of the prefill kernels (kernels/gemm.cu:6-121,
kernels/attn/fast_v2.cu:12-192) against the CPU oracle, through the C ABI.

GEMMs: every output within the fp32 GEMV tolerance (1e-5 relative with the
0.1 * sum|terms| floor, tests/_util.gemv_tol) of the fp64 product with
numpy-dequantized weights, and of the oracle's reference-order fp32 result.
Shapes: Qwen2.5-3B projections (2048 -> 2048, 2048 -> 11008, the Q4_K and
Q6_K 11008 -> 2048 down), K = 896 (floor to 3 super-blocks), ragged column
and token counts, one token.  Attention: every query within 2e-3 absolute of
the fp64 softmax attention over its causal prefix, for head_dim 64/128/256,
GQA, a context already in the cache (pos0 > 0), and the device-pos0 entry.
"""
import numpy as np
import pytest
import torch

import oracle
from taraference_amd import synth
from _gpu import P, S, call, dev, empty, host
from _util import ATTN_ATOL, assert_gemv_close, gemm_ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt,n_rows,n_cols,n_tok", [
    ("q4k", 2048, 2048, 7),
    ("q4k", 2048, 11008, 64),
    ("q4k", 11008, 2048, 33),
    ("q4k", 896, 4864, 5),
    ("q4k", 256, 300, 1),
    ("q4k", 3584, 130, 100),
    ("q6k", 2048, 256, 9),
    ("q6k", 11008, 2048, 17),
    ("q6k", 2048, 4000, 40),
    ("q6k", 256, 77, 2),
])
def test_gemm(gpu, fmt, n_rows, n_cols, n_tok):
    print(f"gemm {fmt} {n_rows}x{n_cols} tok={n_tok}", flush=True)
    rng = np.random.default_rng(n_rows + n_cols + n_tok)
    w, cb = (synth.q4k_matrix if fmt == "q4k" else synth.q6k_matrix)(rng, n_rows, n_cols)
    x = rng.standard_normal((n_tok, n_rows)).astype(np.float32)
    out = empty(n_tok * n_cols)
    call(f"tf_gemm_{fmt}_f32", P(dev(w)), P(dev(x)), P(out), n_rows, n_cols, cb, n_tok, S())
    y = host(out).reshape(n_tok, n_cols)
    ref, absn = gemm_ref(fmt, w, n_rows, x)
    for t in range(n_tok):
        assert_gemv_close(y[t], ref[t], absn[t], f"gemm {fmt} t={t}")
    if n_cols * n_tok * n_rows <= 2048 * 2048 * 8:
        yo = (oracle.gemm_q4k if fmt == "q4k" else oracle.gemm_q6k)(w, x, n_rows, n_cols, cb,
                                                                    n_tok)
        for t in range(n_tok):
            assert_gemv_close(y[t], yo[t].astype(np.float64), absn[t], f"gemm vs oracle t={t}")


@pytest.mark.parametrize("n_head,n_kv,hd,pos0,n_q", [
    (16, 2, 128, 0, 37),    # Qwen2.5-3B heads, a fresh prompt
    (16, 2, 128, 100, 64),  # prompt continued after 100 cached positions
    (14, 2, 64, 0, 200),    # Qwen2.5-0.5B heads
    (4, 1, 256, 5, 20),
    (28, 4, 128, 0, 1),     # Qwen2.5-7B heads, one query
    (16, 2, 128, 1000, 50),  # many key tiles per query block
    (28, 4, 128, 300, 256),  # Qwen2.5-7B heads, a full prompt chunk after 300 positions
])
@pytest.mark.parametrize("junk", ["finite", "nan"])
def test_attn_prefill(gpu, n_head, n_kv, hd, pos0, n_q, junk):
    print(f"attn prefill h={n_head} kv={n_kv} hd={hd} pos0={pos0} n_q={n_q} junk={junk}",
          flush=True)
    rng = np.random.default_rng(n_q * 3 + pos0)
    L = pos0 + n_q
    K = synth.kv_cache(rng, L + 40, n_kv, hd)  # rows past the last query hold junk
    V = synth.kv_cache(rng, L + 40, n_kv, hd)
    if junk == "nan":  # f16 NaN past the last query: must never reach the output
        K[L:] = 0x7E00
        V[L:] = 0x7E00
    q = rng.standard_normal((n_q, n_head * hd)).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(hd)))
    kd, vd, qd = dev(K), dev(V), dev(q)
    out = empty(n_q * n_head * hd)
    call("tf_attn_prefill", P(qd), P(kd), P(vd), P(out), n_head, n_kv, hd, pos0, n_q, scale, S())
    y = host(out).reshape(n_q, -1)
    yo = oracle.attn_prefill(q, K, V, n_head, n_kv, hd, pos0, n_q, scale)
    for qi in range(n_q):
        ref = oracle.attn_f64(q[qi], K, V, n_head, n_kv, hd, pos0 + qi + 1, scale)
        err = np.max(np.abs(y[qi] - ref))
        assert err < ATTN_ATOL, (qi, err)
        assert np.max(np.abs(y[qi] - yo[qi])) < ATTN_ATOL, qi
    p0 = dev(np.array([pos0], np.int32))
    out2 = empty(n_q * n_head * hd)
    call("tf_attn_prefill_d", P(qd), P(kd), P(vd), P(out2), n_head, n_kv, hd, P(p0), n_q, scale,
         S())
    assert np.array_equal(host(out2).reshape(n_q, -1), y)
