"""BASELINE config 4 at its full context: Qwen2.5-7B widths (28 q / 4 kv
heads of 128, hidden 3584, FFN 18944; two layers) with a 32768-token K/V
cache, filled by the runtime's batched prefill (tf_model_prefill), then one
decode step at position 32768 on the multi-launch path (3) and the
persistent path (4).

The CPU reference step (tests/_model_ref.RefModel.step, the oracle's
GEMVs and split-KV flash decode in the reference's order) is given the same
cache rows the GPU prefill wrote, so it checks the decode step itself at
this context: logits within 2e-3 of their RMS for both paths, the new K/V
rows within one f16 ulp plus 1e-2 of the row RMS, and the greedy token equal
to the reference's whenever its top-two gap exceeds the logit tolerance.
"""
import numpy as np
import pytest

from test_gpu_model import build

pytestmark = pytest.mark.gpu

CFG7B = dict(n_layer=2, n_embd=3584, n_ff=18944, n_head=28, n_kv=4, head_dim=128,
             n_vocab=2000, rope_theta=1e6, rms_eps=1e-6)


def test_config4_decode_at_32768(gpu):
    cfg, ctx = CFG7B, 32768
    print(f"config 4 context {ctx}: prefill", flush=True)
    gm, rm = build(cfg, 44, ctx + 8)
    prompt = np.random.default_rng(4).integers(0, cfg["n_vocab"], ctx).tolist()
    tok = gm.prefill(prompt, 0)
    for li in range(cfg["n_layer"]):
        k, v = gm.kv_cache(li, ctx)
        rm.K[li][:ctx] = k
        rm.V[li][:ctx] = v
    print("reference step", flush=True)
    rl, rt = rm.step(tok, ctx)
    scale = np.sqrt(np.mean(rl.astype(np.float64) ** 2))
    top = np.sort(rl)[-2:]
    for path in (3, 4):
        print(f"decode step, path {path}", flush=True)
        gm.set_path(path)
        nxt = gm.forward(tok, ctx)
        lg = gm.logits()
        assert np.abs(lg.astype(np.float64) - rl).max() <= 2e-3 * scale, path
        if top[1] - top[0] > 4e-3 * scale:
            assert nxt == rt, path
        for li in range(cfg["n_layer"]):
            k, v = gm.kv_cache(li, ctx + 1)
            for got, ref in ((k[ctx], rm.K[li][ctx]), (v[ctx], rm.V[li][ctx])):
                r = ref.view(np.float16).astype(np.float64)
                g = got.view(np.float16).astype(np.float64)
                ulp = np.abs(np.spacing(ref.view(np.float16))).astype(np.float64)
                rms = np.sqrt(np.mean(r ** 2))
                assert np.all(np.abs(g - r) <= ulp + 1e-2 * rms), (path, li)
    gm.close()
