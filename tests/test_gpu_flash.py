"""GPU parity of split-KV flash decode (BASELINE config 2 and the 7B GQA
shape) against the oracle and textbook fp64 attention, tolerance 2e-3
absolute.  Also checks the reference's partial-buffer contract (m, l, O) for
empty partitions and the device-position (graph) variant."""
import numpy as np
import pytest
import torch

import oracle
from taraference_amd import capi, synth
from _gpu import P, S, call, dev, empty, host

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def case(L, n_head, n_kv, hd, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    K = synth.kv_cache(rng, L, n_kv, hd)
    V = synth.kv_cache(rng, L, n_kv, hd)
    return q, K, V


def run_gpu(q, K, V, n_head, n_kv, hd, pos0, n_split, scale, device_pos=False):
    part = empty(n_head * n_split * (2 + hd))
    out = empty(n_head * hd)
    qd, kd, vd = dev(q), dev(K), dev(V)
    if device_pos:
        pd = dev(np.array([pos0], np.int32))
        call("tf_flash_decode_partial_d", P(qd), P(kd), P(vd), P(part), n_head, n_kv, hd, P(pd),
             1, n_split, scale, S())
    else:
        call("tf_flash_decode_partial", P(qd), P(kd), P(vd), P(part), n_head, n_kv, hd, pos0, 1,
             n_split, scale, S())
    call("tf_flash_decode_reduce", P(part), P(out), n_head, hd, n_split, 1, S())
    return host(part), host(out)


@pytest.mark.parametrize("L", [1, 5, 512, 777, 4096, 32768])
@pytest.mark.parametrize("split", ["8", "auto"])
def test_flash_config2(gpu, L, split):
    n_head, n_kv, hd = 16, 2, 128
    q, K, V = case(L, n_head, n_kv, hd, L)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    n_split = 8 if split == "8" else capi.load().tf_flash_decode_n_split(n_kv, L)
    part, out = run_gpu(q, K, V, n_head, n_kv, hd, L - 1, n_split, scale)
    ref = oracle.attn_f64(q, K, V, n_head, n_kv, hd, L, scale)
    assert np.abs(out - ref).max() < ATOL
    if n_split == 8 and L <= 4096:
        oref = oracle.flash_reduce(oracle.flash_partial(q, K, V, n_head, n_kv, hd, L - 1, 8, scale),
                                   n_head, hd, 8)
        assert np.abs(out - oref).max() < ATOL
    p = part.reshape(n_head, n_split, 2 + hd)
    chunk = -(-L // n_split)
    empty_s = [s for s in range(n_split) if s * chunk >= L]
    for s in empty_s:
        assert np.all(p[:, s, 0] == np.float32(-1e30)) and np.all(p[:, s, 1:] == 0)


@pytest.mark.parametrize("n_head,n_kv,hd,L", [(28, 4, 128, 3000), (8, 8, 64, 100),
                                              (16, 4, 256, 700)])
def test_flash_shapes(gpu, n_head, n_kv, hd, L):
    q, K, V = case(L, n_head, n_kv, hd, 3)
    scale = 0.09
    _, out = run_gpu(q, K, V, n_head, n_kv, hd, L - 1, 8, scale, device_pos=True)
    ref = oracle.attn_f64(q, K, V, n_head, n_kv, hd, L, scale)
    assert np.abs(out - ref).max() < ATOL


def test_flash_prefix_of_longer_cache(gpu):
    """Attends only positions 0..pos0 of a cache that holds more rows."""
    n_head, n_kv, hd = 16, 2, 128
    q, K, V = case(1024, n_head, n_kv, hd, 11)
    _, out = run_gpu(q, K, V, n_head, n_kv, hd, 600, 8, 0.088)
    ref = oracle.attn_f64(q, K[:601].copy(), V[:601].copy(), n_head, n_kv, hd, 601, 0.088)
    assert np.abs(out - ref).max() < ATOL


@pytest.mark.parametrize("n_head,n_kv,hd,L,n_split", [
    (16, 2, 128, 1, 8), (16, 2, 128, 5, 8), (16, 2, 128, 777, 8), (16, 2, 128, 4096, 32),
    (16, 2, 128, 5000, 64), (16, 2, 128, 32768, 256),
    (28, 4, 128, 3000, 16), (8, 8, 64, 100, 8), (32, 2, 128, 600, 8), (16, 4, 256, 700, 24),
    (16, 2, 128, 1, 1), (16, 2, 128, 512, 1), (16, 2, 128, 2048, 1), (28, 4, 128, 3000, 1),
    (8, 8, 64, 100, 1)])
def test_flash_decode_one_call(gpu, n_head, n_kv, hd, L, n_split):
    """tf_flash_decode: split partials then the log-sum-exp merge (+ Q8 of
    the merged output) in one call.  Attention within 2e-3 of fp64 softmax
    attention, the Q8 bit-exact against quantizing the f32 it wrote, and
    the per-kv-head counters still zero after each call (two calls in a
    row give the same result; the second reads the position from device
    memory)."""
    q, K, V = case(L, n_head, n_kv, hd, L + n_split)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    part = empty(n_head * n_split * (2 + hd))
    cnt = torch.zeros(n_kv, dtype=torch.int32, device="cuda")
    qd, kd, vd = dev(q), dev(K), dev(V)
    outs = []
    for call_no in range(2):
        out, q8, d8 = empty(n_head * hd), empty(n_head * hd, torch.int8), empty(n_head * hd // 32)
        pd = dev(np.array([L - 1], np.int32)) if call_no else None
        call("tf_flash_decode", P(qd), P(kd), P(vd), P(part), P(cnt), P(out), P(q8), P(d8),
             n_head, n_kv, hd, L - 1 if call_no == 0 else 0, P(pd), n_split, scale, S())
        o = host(out)
        assert not host(cnt).any()
        rq, rd = oracle.quantize_q8(o)
        assert np.array_equal(host(q8), rq)
        assert np.array_equal(host(d8).view(np.uint32), rd.view(np.uint32))
        outs.append(o)
    ref = oracle.attn_f64(q, K, V, n_head, n_kv, hd, L, scale)
    assert np.abs(outs[0] - ref).max() < ATOL
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("n_head,n_kv,L", [(16, 2, 512), (16, 2, 1500), (28, 4, 777)])
def test_flash_single_partition_direct_output(gpu, n_head, n_kv, L):
    """With one partition tf_flash_decode writes the output (and its Q8) from
    the partial kernel itself: bit-identical to the partial + merge pair of
    launches (tf_flash_decode_partial, tf_flash_decode_reduce_q8)."""
    hd = 128
    q, K, V = case(L, n_head, n_kv, hd, L + 1)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    qd, kd, vd = dev(q), dev(K), dev(V)
    n = n_head * hd
    part = empty(n_head * (2 + hd))
    o1, q1, d1 = empty(n), empty(n, torch.int8), empty(n // 32)
    call("tf_flash_decode", P(qd), P(kd), P(vd), P(part), None, P(o1), P(q1), P(d1),
         n_head, n_kv, hd, L - 1, None, 1, scale, S())
    o2, q2, d2 = empty(n), empty(n, torch.int8), empty(n // 32)
    call("tf_flash_decode_partial", P(qd), P(kd), P(vd), P(part), n_head, n_kv, hd, L - 1, 1, 1,
         scale, S())
    call("tf_flash_decode_reduce_q8", P(part), P(o2), P(q2), P(d2), n_head, hd, 1, S())
    assert np.array_equal(host(o1).view(np.uint32), host(o2).view(np.uint32))
    assert np.array_equal(host(q1), host(q2))
    assert np.array_equal(host(d1).view(np.uint32), host(d2).view(np.uint32))
    ref = oracle.attn_f64(q, K, V, n_head, n_kv, hd, L, scale)
    assert np.abs(host(o1) - ref).max() < ATOL
