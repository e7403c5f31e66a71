"""Oracle pins for split-KV flash decode (kernels/attn/flash.cu:16-255).

Pins: agreement with textbook softmax attention in fp64 over the same f16
cache (numpy, independent of the oracle's C loops), seq_len = 1 -> out = V0,
q = 0 (uniform weights) -> mean of V over the context, and independence of
the result from the number of partitions (including empty partitions).
"""
import numpy as np
import pytest

import oracle
from taraference_amd import synth

ATOL = 2e-3


def np_attn(q, K, V, n_head, n_kv, hd, L, scale):
    Kf = K[:L].view(np.float16).astype(np.float64).reshape(L, n_kv, hd)
    Vf = V[:L].view(np.float16).astype(np.float64).reshape(L, n_kv, hd)
    qf = q.astype(np.float64).reshape(n_head, hd)
    out = np.zeros((n_head, hd))
    rep = n_head // n_kv
    for h in range(n_head):
        s = Kf[:, h // rep] @ qf[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ Vf[:, h // rep]
    return out.reshape(-1)


def run(q, K, V, n_head, n_kv, hd, L, n_split, scale):
    part = oracle.flash_partial(q, K, V, n_head, n_kv, hd, L - 1, n_split, scale)
    return oracle.flash_reduce(part, n_head, hd, n_split)


@pytest.mark.parametrize("L,n_split", [(1, 8), (7, 8), (512, 8), (1000, 8), (1000, 3), (4096, 8)])
def test_flash_vs_textbook(L, n_split):
    n_head, n_kv, hd = 16, 2, 128
    rng = np.random.default_rng(L)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    K = synth.kv_cache(rng, L, n_kv, hd)
    V = synth.kv_cache(rng, L, n_kv, hd)
    scale = float(np.float32(1.0 / np.sqrt(hd)))  # the kernels take an f32 scale
    out = run(q, K, V, n_head, n_kv, hd, L, n_split, scale)
    ref = np_attn(q, K, V, n_head, n_kv, hd, L, scale)
    assert np.abs(out - ref).max() < ATOL
    ref64 = oracle.attn_f64(q, K, V, n_head, n_kv, hd, L, scale)
    assert np.allclose(ref64, ref, atol=1e-12)


def test_flash_l1_is_v0():
    n_head, n_kv, hd = 8, 2, 128
    rng = np.random.default_rng(0)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    K = synth.kv_cache(rng, 1, n_kv, hd)
    V = synth.kv_cache(rng, 1, n_kv, hd)
    out = run(q, K, V, n_head, n_kv, hd, 1, 8, 0.1).reshape(n_head, hd)
    v0 = V[0].view(np.float16).astype(np.float32).reshape(n_kv, hd)
    for h in range(n_head):
        assert np.array_equal(out[h], v0[h // 4])


def test_flash_uniform_is_mean():
    n_head, n_kv, hd, L = 4, 1, 64, 300
    rng = np.random.default_rng(1)
    q = np.zeros(n_head * hd, np.float32)
    K = synth.kv_cache(rng, L, n_kv, hd)
    V = synth.kv_cache(rng, L, n_kv, hd)
    out = run(q, K, V, n_head, n_kv, hd, L, 8, 1.0).reshape(n_head, hd)
    mean = V.view(np.float16).astype(np.float64).mean(0)
    assert np.abs(out - mean[None, :]).max() < 1e-5


def test_flash_split_invariance_and_empty_partitions():
    n_head, n_kv, hd, L = 16, 2, 128, 5   # 8 splits of 1 token: 3 are empty
    rng = np.random.default_rng(2)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    K = synth.kv_cache(rng, L, n_kv, hd)
    V = synth.kv_cache(rng, L, n_kv, hd)
    part = oracle.flash_partial(q, K, V, n_head, n_kv, hd, L - 1, 8, 0.2)
    p = part.reshape(n_head, 8, 2 + hd)
    assert np.all(p[:, 5:, 0] == np.float32(-1e30)) and np.all(p[:, 5:, 1:] == 0)
    a = oracle.flash_reduce(part, n_head, hd, 8)
    b = run(q, K, V, n_head, n_kv, hd, L, 1, 0.2)
    assert np.abs(a - b).max() < 1e-5
