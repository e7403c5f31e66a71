"""The planted Q8 near-tie inputs (tests/q8_ties.py) really sit at the
rounding boundaries, so the GPU tests that use them exercise the
reciprocal-quotient fix-up of the in-kernel quantizers."""
import numpy as np

import oracle
from q8_ties import near_tie_groups


def test_near_ties_hit_the_boundary():
    x = near_tie_groups(256, 1)
    g = x.reshape(-1, 32)
    amax = np.abs(g).max(axis=1)
    d = (amax * (np.float32(1) / np.float32(127))).astype(np.float32)
    live = amax > 0
    z = g[live].astype(np.float64) / d[live, None].astype(np.float64)
    frac = np.abs(np.abs(z) - np.floor(np.abs(z)) - 0.5)
    near = frac < 2.0 ** -14
    assert near[:, 1:].mean() > 0.9, "planted values are not near a .5 tie"
    q, dq = oracle.quantize_q8(x)
    qq = q.reshape(-1, 32)[live].astype(np.float64)
    # both directions occur: rounded up and down at the tie
    up = (np.abs(qq) > np.abs(z) + 1e-12) & near
    down = (np.abs(qq) < np.abs(z) - 1e-12) & near
    assert up.sum() > 100 and down.sum() > 100
    assert (~live).sum() >= 32 and np.all(q.reshape(-1, 32)[~live] == 0)
    assert np.all(dq[~live] == 0)
    assert np.any((dq > 0) & (dq < np.float32(1.17549435e-38)))  # subnormal scales
