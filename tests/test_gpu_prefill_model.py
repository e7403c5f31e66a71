"""The runtime's batched prompt forward (tf_model_prefill: forward.rs:42-71
with the n_tok-row layer of layer.rs) against the CPU reference prefill
(tests/_model_ref.RefModel.prefill: oracle f32 GEMMs, prefill attention,
rope, RMSNorm rows) on tiny random-init Qwen2-shaped Q4_K_M models.

Both sides run fp32 activations through the same operator sequence and
differ only in fp32 summation order.  The K/V rows agree to one f16 ulp plus
2e-4 of the row RMS in layer 0 (the GEMM bound, 1e-5 of sum |terms|, with
sum |terms| about sqrt(K) = 16 row RMS for these rows) and 1e-3 of the row
RMS after it.  The last token's logits (the decode head: RMSNorm, Q8,
lm_head) agree to 5e-3 of their RMS: the hidden row carries the order
differences of every layer (up to 1e-3 of RMS each, as the K/V bound), and
quantizing it to Q8 can flip a value by one step, which moves the logits by
about d8 |w|.  The returned token equals the reference's argmax whenever its
top-two gap exceeds 1e-2 of the RMS.  Prompts cross the 256-token chunk boundary, and a second
prefill continues at pos0 > 0.  The greedy continuation after a prefill
starts with prefill's token and runs on the decode path.
"""
import numpy as np
import pytest

from test_gpu_model import TINY, build

pytestmark = pytest.mark.gpu


def f16(a):
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float64)


def check_kv(gm, rm, n_layer, rows):
    for li in range(n_layer):
        gk, gv = gm.kv_cache(li, rows.stop)
        for got, ref in ((gk, rm.K[li]), (gv, rm.V[li])):
            g, r = f16(got[rows]), f16(ref[rows])
            rms = np.sqrt(np.mean(r ** 2, axis=1, keepdims=True))
            ulp = np.abs(r) * 2.0 ** -10 + 2.0 ** -24
            rel = 2e-4 if li == 0 else 1e-3
            assert np.all(np.abs(g - r) <= ulp + rel * rms), (li, np.max(np.abs(g - r) / rms))


def check_logits(gm, ref_logits, ref_tok, tok):
    lg = gm.logits().astype(np.float64)
    rl = ref_logits.astype(np.float64)
    scale = np.sqrt(np.mean(rl ** 2))
    assert np.max(np.abs(lg - rl)) <= 5e-3 * scale
    top = np.sort(rl)[-2:]
    if top[1] - top[0] > 1e-2 * scale:
        assert tok == ref_tok


@pytest.mark.parametrize("ci,n_prompt,n_more", [(0, 300, 21), (1, 40, 7), (2, 37, 0)])
def test_prefill_matches_reference(gpu, ci, n_prompt, n_more):
    cfg = TINY[ci]
    print(f"prefill model cfg {ci} n={n_prompt}+{n_more}", flush=True)
    max_seq = n_prompt + n_more + 8
    gm, rm = build(cfg, 300 + ci, max_seq)
    rng = np.random.default_rng(7 + ci)
    prompt = rng.integers(0, cfg["n_vocab"], n_prompt + n_more).tolist()
    tok = gm.prefill(prompt[:n_prompt], 0)
    rl, rt = rm.prefill(prompt[:n_prompt], 0)
    check_kv(gm, rm, cfg["n_layer"], slice(0, n_prompt))
    check_logits(gm, rl, rt, tok)
    if n_more:
        tok2 = gm.prefill(prompt[n_prompt:], n_prompt)
        rl2, rt2 = rm.prefill(prompt[n_prompt:], n_prompt)
        check_kv(gm, rm, cfg["n_layer"], slice(0, n_prompt + n_more))
        check_logits(gm, rl2, rt2, tok2)
    gm.close()


def test_generate_after_prefill(gpu):
    cfg = TINY[0]
    gm, _ = build(cfg, 400, 64)
    prompt = np.random.default_rng(3).integers(0, cfg["n_vocab"], 20).tolist()
    out = gm.generate_prefilled(prompt, 6)
    assert len(out) == 6
    # the first token is prefill's; the rest continue on the decode path
    first = gm.prefill(prompt, 0)
    assert out[0] == first
    rest = gm.generate([first], 5, pos0=len(prompt))
    assert list(out[1:]) == list(rest)
    gm.close()
