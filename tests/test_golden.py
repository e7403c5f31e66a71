"""The committed fixtures of tests/golden/ (written by make_golden.py).

CPU: the oracle still reproduces every fixture bit for bit, and each fp32
result is within the parity tolerance of the fixture's fp64 truth.
GPU: the HIP library, called through the C ABI, matches each fixture to the
parity bar: Q8 bytes and scales bit-exact, GEMV outputs within 1e-5
relative (tests/_util.gemv_tol), attention within 2e-3 absolute.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from _util import assert_ffn_close, assert_gemv_close

GOLDEN = Path(__file__).resolve().parent / "golden"
Q8_FILES = ["q8_k896", "q8_k2048", "q8_k3584", "q8_k11008"]


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def same_bits(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and np.array_equal(
        np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


# ------------------------------------------------------------------ CPU

@pytest.mark.parametrize("name", Q8_FILES)
def test_oracle_reproduces_q8(name):
    g = load(name)
    q8, d8 = oracle.quantize_q8(g["x"])
    assert same_bits(q8, g["q8"]) and same_bits(d8, g["d8"])
    assert not g["q8"][:32].any() and g["d8"][0] == 0          # all-zero group


def test_oracle_reproduces_gemv_q4k_k896():
    g = load("gemv_q4k_k896")
    y = oracle.gemv_q4k_q8(g["w"], g["xq"], g["xd"], 896, g["w"].shape[0], int(g["col_bytes"]))
    assert same_bits(y, g["y"])
    assert_gemv_close(g["y"], g["y64"], g["rowabs"], "golden q4k")


def test_oracle_reproduces_ffn():
    g = load("ffn_q4k_k2048")
    n = g["gate"].shape[0]
    h = oracle.gemv_q4k_ffn(g["gate"], g["up"], g["xq"], g["xd"], 2048, n, int(g["col_bytes"]))
    assert same_bits(h, g["h"])
    assert_ffn_close(g["h"], g["g64"], g["ga"], g["u64"], g["ua"], "golden ffn")


def test_oracle_reproduces_down_q6k():
    g = load("down_q6k_k11008")
    n = g["w"].shape[0]
    y = oracle.gemv_q6k_compact_q8_kway(g["w"], g["xq"], g["xd"], 11008, n, int(g["col_bytes"]),
                                        8, use_res=2, out=g["residual"])
    assert same_bits(y, g["y"])
    assert_gemv_close(g["y"] - g["residual"], g["y64"], g["rowabs"], "golden q6k")


def test_oracle_reproduces_flash():
    g = load("flash_L130")
    L = g["k"].shape[0]
    part = oracle.flash_partial(g["q"], g["k"], g["v"], 16, 2, 128, L - 1, 8, float(g["scale"]))
    out = oracle.flash_reduce(part, 16, 128, 8)
    assert same_bits(out, g["out"])
    assert np.max(np.abs(g["out"] - g["out64"])) < 2e-3


# ------------------------------------------------------------------ GPU

@pytest.mark.gpu
@pytest.mark.parametrize("name", Q8_FILES)
def test_gpu_q8_golden(gpu, name):
    from _gpu import P, S, call, dev, empty, host
    g = load(name)
    n = g["x"].size
    q8, d8 = empty(n, torch.int8), empty(n // 32)
    call("tf_quantize_q8", P(dev(g["x"])), P(q8), P(d8), n, S())
    assert same_bits(host(q8), g["q8"]) and same_bits(host(d8), g["d8"])


@pytest.mark.gpu
def test_gpu_gemv_q4k_golden(gpu):
    from _gpu import P, S, call, dev, empty, host
    g = load("gemv_q4k_k896")
    n = g["w"].shape[0]
    y = empty(n)
    call("tf_gemv_q4k_q8", P(dev(g["w"])), P(dev(g["xq"])), P(dev(g["xd"])), P(y), 896, n,
         int(g["col_bytes"]), 0, None, 0, None, S())
    assert_gemv_close(host(y), g["y64"], g["rowabs"], "gpu golden q4k")
    assert_gemv_close(host(y), g["y"].astype(np.float64), g["rowabs"], "gpu vs oracle q4k")


@pytest.mark.gpu
def test_gpu_ffn_golden(gpu):
    from _gpu import P, S, call, dev, empty, host
    g = load("ffn_q4k_k2048")
    n = g["gate"].shape[0]
    h = empty(n)
    call("tf_gemv_q4k_ffn", P(dev(g["gate"])), P(dev(g["up"])), P(dev(g["xq"])),
         P(dev(g["xd"])), P(h), 2048, n, int(g["col_bytes"]), S())
    assert_ffn_close(host(h), g["g64"], g["ga"], g["u64"], g["ua"], "gpu golden ffn")


@pytest.mark.gpu
def test_gpu_down_q6k_golden(gpu):
    from _gpu import P, S, call, dev, empty, host
    g = load("down_q6k_k11008")
    n = g["w"].shape[0]
    y = dev(g["residual"].copy())
    call("tf_gemv_q6k_down_splitk", P(dev(g["w"])), P(dev(g["xq"])), P(dev(g["xd"])), P(y),
         11008, n, int(g["col_bytes"]), 0, None, 2, None, S())
    assert_gemv_close(host(y) - g["residual"], g["y64"], g["rowabs"], "gpu golden q6k")


@pytest.mark.gpu
def test_gpu_flash_golden(gpu):
    from _gpu import P, S, call, dev, empty, host
    g = load("flash_L130")
    L = g["k"].shape[0]
    part, out = empty(16 * 8 * 130), empty(16 * 128)
    call("tf_flash_decode_partial", P(dev(g["q"])), P(dev(g["k"])), P(dev(g["v"])), P(part), 16,
         2, 128, L - 1, 1, 8, float(g["scale"]), S())
    call("tf_flash_decode_reduce", P(part), P(out), 16, 128, 8, 1, S())
    o = host(out)
    assert np.max(np.abs(o - g["out"])) < 2e-3
    assert np.max(np.abs(o - g["out64"])) < 2e-3
