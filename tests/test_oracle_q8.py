"""Oracle pins for the Q8 activation quantize (kernels/gemv.cu:43-65).

Pins: the closed form d = amax * fl(1/127), q = rint_even(x / d) with IEEE
division (checked against numpy's float32 arithmetic), |q| <= 127, the amax
element mapping to +-127, all-zero groups, reconstruction error <= d/2, and
exact ties rounding to even.
"""
import numpy as np
import pytest

import oracle


def np_quant(x):
    x = x.astype(np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax * np.float32(1.0 / 127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(amax[:, None] == 0, 0, np.rint(x / d[:, None]))
    return q.astype(np.int8).reshape(-1), d


@pytest.mark.parametrize("n", [32, 896, 2048, 3584, 11008, 18944])
def test_q8_closed_form(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    q, d = oracle.quantize_q8(x)
    q_np, d_np = np_quant(x)
    assert np.array_equal(q, q_np)
    assert np.array_equal(d.view(np.uint32), d_np.view(np.uint32))


def test_q8_invariants():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(4096) * rng.uniform(1e-3, 1e3, 4096)).astype(np.float32)
    x[:32] = 0.0  # all-zero group
    q, d = oracle.quantize_q8(x)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    assert np.all(q[:32] == 0) and d[0] == 0.0
    g = x.reshape(-1, 32)
    qg = q.reshape(-1, 32)
    am = np.argmax(np.abs(g), axis=1)
    for i in range(1, g.shape[0]):
        assert abs(int(qg[i, am[i]])) == 127
        assert np.sign(qg[i, am[i]]) == np.sign(g[i, am[i]])
    err = np.abs(qg.astype(np.float64) * d[:, None] - g)
    assert np.all(err <= d[:, None].astype(np.float64) * 0.5 * (1 + 1e-6))


def test_q8_ties_round_to_even():
    # choose amax so that d is a power of two: then k + 0.5 ties are exact
    amax = np.float32(127.0)
    d = np.float32(amax * np.float32(1.0 / 127.0))
    x = np.zeros(32, np.float32)
    x[0] = amax
    ties = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 100.5], np.float32) * d
    x[1:9] = ties
    q, dd = oracle.quantize_q8(x)
    assert dd[0] == d == np.float32(1.0)  # exact ties below
    exp = np.rint(ties.astype(np.float64) / float(d)).astype(np.int8)  # half-even
    assert np.array_equal(q[1:9], exp)
