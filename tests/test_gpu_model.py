"""GPU decode-step runtime against the CPU reference step (tests/_model_ref.py)
on tiny random-init Qwen2-shaped models in the Q4_K_M mix.

Checks, per step: in layer 0 (whose input, the embedding row, and its
RMSNorm + Q8 are bit-identical on both sides) the appended f16 K/V rows are
within one f16 ulp plus the fp32 GEMV tolerance (1e-5 of the row RMS, the
cancellation floor) of the reference's; in later layers, whose inputs carry
the fp32 differences of earlier GEMVs and so may take a one-step Q8 rounding
flip, within 1e-2 of the row RMS (a flip moves every output of the GEMV by
d8 * w, about 1e-3 of the row RMS); the logits agree to a relative 2e-3 of their RMS (the
per-op fp32 differences plus occasional one-step Q8 rounding flips of
intermediate activations), and the greedy token is equal whenever the
reference's top-two logit gap exceeds that tolerance.  The HIP-graph
replay path must produce exactly the tokens of the eager device-state path.
"""
import numpy as np
import pytest

from taraference_amd import synth
from _model_ref import RefModel

pytestmark = pytest.mark.gpu

TINY = [
    dict(n_layer=2, n_embd=256, n_ff=512, n_head=2, n_kv=1, head_dim=128, n_vocab=300,
         rope_theta=1e6, rms_eps=1e-6),
    dict(n_layer=3, n_embd=512, n_ff=768, n_head=4, n_kv=2, head_dim=128, n_vocab=1000,
         rope_theta=1e4, rms_eps=1e-6),
    # the real 3B and 7B widths (two layers, small vocabulary)
    dict(n_layer=2, n_embd=2048, n_ff=11008, n_head=16, n_kv=2, head_dim=128, n_vocab=2000,
         rope_theta=1e6, rms_eps=1e-6),
    dict(n_layer=2, n_embd=3584, n_ff=18944, n_head=28, n_kv=4, head_dim=128, n_vocab=2000,
         rope_theta=1e6, rms_eps=1e-6),
]


def build(cfg, seed, max_seq):
    from taraference_amd.model import DecodeModel

    rng = np.random.default_rng(seed)
    layers = [synth.qwen_layer(rng, cfg, li) for li in range(cfg["n_layer"])]
    emb = synth.qwen_embedding(rng, cfg)
    c = dict(cfg, max_seq=max_seq)
    return DecodeModel(c, layers, emb), RefModel(cfg, layers, emb, max_seq)


@pytest.mark.parametrize("path", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("ci", [0, 1, 2, 3])
def test_decode_steps_match_reference(gpu, ci, path):
    cfg = TINY[ci]
    gm, rm = build(cfg, 100 + ci, 48)
    gm.set_path(path)
    rng = np.random.default_rng(ci)
    prompt = rng.integers(0, cfg["n_vocab"], 12).tolist()
    tok = prompt[0]
    for pos in range(24):
        nxt = gm.forward(tok, pos)
        lg = gm.logits()
        rl, rt = rm.step(tok, pos)
        scale = np.sqrt(np.mean(rl.astype(np.float64) ** 2))
        err = np.abs(lg - rl).max()
        assert err <= 2e-3 * scale, (pos, err, scale)
        srt = np.sort(rl)
        if srt[-1] - srt[-2] > 2e-3 * scale:
            assert nxt == rt, pos
        for li in range(cfg["n_layer"]):
            K, V = gm.kv_cache(li, pos + 1)
            for got, ref in ((K[pos], rm.K[li][pos]), (V[pos], rm.V[li][pos])):
                g = got.view(np.float16).astype(np.float64)
                r = ref.view(np.float16).astype(np.float64)
                ulp = np.abs(np.spacing(ref.view(np.float16))).astype(np.float64)
                rms = np.sqrt(np.mean(r ** 2))
                tol = ulp + (1e-5 if li == 0 else 1e-2) * rms
                assert np.all(np.abs(g - r) <= tol), (li, pos, np.abs(g - r).max())
        tok = prompt[pos + 1] if pos + 1 < len(prompt) else rt
    gm.close()


@pytest.mark.parametrize("path", [0, 1, 2, 3, 4])
def test_graph_replay_equals_eager(gpu, path):
    cfg = TINY[1]
    gm, _ = build(cfg, 7, 64)
    gm.set_path(path)
    prompt = list(range(5, 21))
    eager = gm.generate(prompt, 20, use_graph=False)
    graph = gm.generate(prompt, 20, use_graph=True)
    again = gm.generate(prompt, 20, use_graph=True)
    assert np.array_equal(eager, graph) and np.array_equal(graph, again)
    # the same continuation from single eager steps
    tok, toks = prompt[0], []
    for pos in range(len(prompt) + 19):
        nxt = gm.forward(tok, pos)
        if pos >= len(prompt) - 1:
            toks.append(nxt)
        tok = prompt[pos + 1] if pos + 1 < len(prompt) else nxt
    assert np.array_equal(np.array(toks[:20]), eager)
    gm.close()
