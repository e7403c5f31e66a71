"""The persistent decode step's in-kernel quantizers (the eight-lane staging
of its RMSNorm outputs and the sixteen-lane quantization of the attention
output and of h), driven through tf_decode_step_quantize_q8 on inputs
planted at the rounding boundaries, against quantize_q8_global
(kernels/gemv.cu:43-65, the oracle) byte for byte, and against the
standalone tf_quantize_q8."""
import numpy as np
import pytest
import torch

import oracle
from _gpu import P, S, call, dev, empty, host
from q8_ties import near_tie_groups

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("variant", [0, 1], ids=["norm_staging", "pair16"])
@pytest.mark.parametrize("n_groups", [8, 344, 4096])
def test_step_quantizer_bit_exact(gpu, variant, n_groups):
    x = near_tie_groups(n_groups, 17 + n_groups)
    n = x.size
    q, d = empty(n, torch.int8), empty(n // 32)
    call("tf_decode_step_quantize_q8", P(dev(x)), n, variant, P(q), P(d), S())
    q_ref, d_ref = oracle.quantize_q8(x)
    gq, gd = host(q), host(d)
    bad = np.nonzero(gq != q_ref)[0]
    assert bad.size == 0, (f"{bad.size} values differ, first i={bad[0]} x={x[bad[0]]!r} "
                           f"q={gq[bad[0]]} ref={q_ref[bad[0]]}")
    assert np.array_equal(gd.view(np.uint32), d_ref.view(np.uint32))
    # the standalone quantizer agrees too
    q2, d2 = empty(n, torch.int8), empty(n // 32)
    call("tf_quantize_q8", P(dev(x)), P(q2), P(d2), n, S())
    assert np.array_equal(host(q2), q_ref)
    assert np.array_equal(host(d2).view(np.uint32), d_ref.view(np.uint32))


def test_step_quantizer_rejects(gpu):
    x = empty(64)
    q, d = empty(64, torch.int8), empty(2)
    from taraference_amd import capi
    lib = capi.load()
    assert lib.tf_decode_step_quantize_q8(P(x), 48, 0, P(q), P(d), S()) != 0
    assert lib.tf_decode_step_quantize_q8(P(x), 64, 2, P(q), P(d), S()) != 0
