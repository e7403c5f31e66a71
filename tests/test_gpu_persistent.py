"""The persistent decode step (path 4: one launch per token, device-wide
barriers between stages) against the multi-launch fused path (path 3) at
contexts long enough to split the KV cache over several workgroups per kv
head, whose partials the last workgroup merges (log-sum-exp,
attn/flash.cu:222-255).

Both paths run on the same model object, so they read the same weights; each
regenerates the whole K/V cache from the same forced prompt.  Bars: the
logits of the last step within 2e-3 of their RMS, the K/V rows of every
position within one f16 ulp plus 1e-2 of the row RMS (the tolerance of the
per-step reference test for layers past the first), and the greedy token
equal when the fused path's top-two logit gap exceeds the logit tolerance.
Layer 0 must match everywhere.  Past it, at most one position per thousand
may exceed the row bound: at these contexts the synthetic weights make the
scores huge (|q.k| scale ~ 1e5), so the softmax is nearly one-hot and the
fp32 summation order of a score (the two paths differ) can reorder a
near-tie between the top tokens of a position, which moves that position's
attention output -- and so the next layer's K/V row -- by up to a quarter
of its RMS.  The logits of the final step must still agree.
A second persistent run over the same prompt must reproduce the first bit
for bit (every reduction order is fixed).
"""
import numpy as np
import pytest

from taraference_amd import synth

pytestmark = pytest.mark.gpu

CFGS = {
    "3b": dict(n_layer=2, n_embd=2048, n_ff=11008, n_head=16, n_kv=2, head_dim=128,
               n_vocab=2000, rope_theta=1e6, rms_eps=1e-6),
    "7b": dict(n_layer=2, n_embd=3584, n_ff=18944, n_head=28, n_kv=4, head_dim=128,
               n_vocab=2000, rope_theta=1e6, rms_eps=1e-6),
}


def _build(cfg, seed, max_seq):
    from taraference_amd.model import DecodeModel

    rng = np.random.default_rng(seed)
    layers = [synth.qwen_layer(rng, cfg, li) for li in range(cfg["n_layer"])]
    emb = synth.qwen_embedding(rng, cfg)
    return DecodeModel(dict(cfg, max_seq=max_seq), layers, emb)


def _kv(gm, n_layer, seq):
    return [tuple(np.array(a) for a in gm.kv_cache(li, seq)) for li in range(n_layer)]


@pytest.mark.parametrize("name,ctx", [("3b", 700), ("3b", 4100), ("7b", 9000)])
def test_persistent_matches_fused_long_context(gpu, name, ctx):
    cfg = CFGS[name]
    print(f"persistent long-context case {name} ctx={ctx}", flush=True)
    gm = _build(cfg, 11, ctx + 8)
    rng = np.random.default_rng(ctx)
    prompt = rng.integers(0, cfg["n_vocab"], ctx).tolist()
    out = {}
    for key, path in (("fused", 3), ("p0", 4), ("p1", 4)):
        gm.set_path(path)
        toks = gm.generate(prompt, 1)
        out[key] = (np.array(toks), gm.logits(), _kv(gm, cfg["n_layer"], ctx))
    gm.close()
    t3, l3, kv3 = out["fused"]
    t4, l4, kv4 = out["p0"]
    # the persistent step is deterministic: fixed reduction orders everywhere
    _, l4b, kv4b = out["p1"]
    assert np.array_equal(l4, l4b)
    for (ka, va), (kb, vb) in zip(kv4, kv4b):
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    scale = np.sqrt(np.mean(l3.astype(np.float64) ** 2))
    assert np.abs(l4 - l3).max() <= 2e-3 * scale
    for li, ((k3, v3), (k4, v4)) in enumerate(zip(kv3, kv4)):
        for got, ref in ((k4, k3), (v4, v3)):
            r = ref.view(np.float16).astype(np.float64)
            g = got.view(np.float16).astype(np.float64)
            ulp = np.abs(np.spacing(ref.view(np.float16))).astype(np.float64)
            rms = np.sqrt(np.mean(r ** 2, axis=1, keepdims=True))
            bad = np.nonzero(~np.all(np.abs(g - r) <= ulp + 1e-2 * rms, axis=1))[0]
            if li == 0:
                assert bad.size == 0, bad[:8]
            else:
                assert bad.size <= max(1, ctx // 1000), bad[:8]
    srt = np.sort(l3)
    if srt[-1] - srt[-2] > 2e-3 * scale:
        assert t4[0] == t3[0]
