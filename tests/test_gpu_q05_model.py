"""A Qwen2.5-0.5B-layout model (hidden 896, not a multiple of 256, so its
896-row matrices are Q5_0 / Q8_0 as in real Q4_K_M files; ffn_down Q4_K /
Q6_K; a tied Q8_0 embedding) written as a GGUF file, loaded with
DecodeModel.from_gguf and decoded by the runtime's reference operator
sequence (path 0, the only path for these formats), against the CPU
reference step RefModelMixed (the oracle's Q5_0 / Q8_0 / K-quant GEMVs in the
same kernel choices).

Bars: the new K/V rows within one f16 ulp plus 2e-4 of the row RMS in layer
0 (Q5_0 is an fp32 GEMV: 1e-5 of sum |terms|, about 16 row RMS here) and
1e-2 after it.  Logits within 2e-3 of their RMS plus four one-step Q8 flips
of the lm_head input: the last hidden row carries fp32 order differences,
and where one of its values sits at a Q8 rounding boundary the two sides
round it to neighbouring steps, which moves every logit by up to
d8 * max|W| (d8 the group's scale; the synthetic Q8_0 table has |W| up to
1.27, about 2e-3 of the logit RMS per flip).  The greedy token equal
whenever the reference's top-two gap exceeds the logit tolerance.
"""
import numpy as np
import pytest

import _gguf_write as W
import oracle
from taraference_amd import synth
from _util import q8_0_dequant
from _model_ref import RefModelMixed

pytestmark = pytest.mark.gpu

CFG = dict(n_layer=2, n_embd=896, n_ff=4864, n_head=14, n_kv=2, head_dim=64, n_vocab=1000,
           rope_theta=1e6, rms_eps=1e-6)


def write_model(path, cfg, layers, emb):
    meta = W.model_meta(cfg)
    t = []

    def mat(name, wm, n_rows):
        w, cb, ty = wm
        assert cb == W.nbytes(ty, n_rows)
        t.append((name, [n_rows, w.shape[0]], ty, np.ascontiguousarray(w).tobytes()))

    def vec(name, v):
        t.append((name, [len(v)], 0, np.asarray(v, np.float32).tobytes()))

    e = cfg["n_embd"]
    mat("token_embd.weight", emb, e)
    vec("output_norm.weight", np.ones(e, np.float32))
    for i, L in enumerate(layers):
        p = f"blk.{i}"
        vec(f"{p}.attn_norm.weight", L["attn_norm"])
        vec(f"{p}.ffn_norm.weight", L["ffn_norm"])
        mat(f"{p}.attn_q.weight", L["wq"], e)
        mat(f"{p}.attn_k.weight", L["wk"], e)
        mat(f"{p}.attn_v.weight", L["wv"], e)
        for k in ("bq", "bk", "bv"):
            vec(f"{p}.attn_{k[1]}.bias", L[k])
        mat(f"{p}.attn_output.weight", L["wo"], cfg["n_head"] * cfg["head_dim"])
        mat(f"{p}.ffn_gate.weight", L["gate"], e)
        mat(f"{p}.ffn_up.weight", L["up"], e)
        mat(f"{p}.ffn_down.weight", L["down"], cfg["n_ff"])
    W.write(path, meta, t)


def f16(a):
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float64)


def test_q05_layout_decode_matches_reference(gpu, tmp_path):
    from taraference_amd import capi
    from taraference_amd.model import DecodeModel

    cfg = CFG
    rng = np.random.default_rng(505)
    layers = [synth.qwen05_layer(rng, cfg, li) for li in range(cfg["n_layer"])]
    emb = synth.qwen05_embedding(rng, cfg)
    path = tmp_path / "q05.gguf"
    write_model(path, cfg, layers, emb)
    max_seq = 40
    gm = DecodeModel.from_gguf(path, max_seq)
    assert gm.path() == 0
    for p in (1, 3, 4):
        with pytest.raises(capi.HipError):
            gm.set_path(p)
    with pytest.raises(capi.HipError):  # prefill is for the K-quant placement
        gm.prefill([1, 2, 3], 0)
    rm = RefModelMixed(cfg, layers, emb, max_seq)
    nb = cfg["n_embd"] // 32
    wmax = float(np.abs(q8_0_dequant(emb[0][:, : nb * 34].reshape(-1, 34))).max())
    prompt = np.random.default_rng(6).integers(0, cfg["n_vocab"], 10).tolist()
    tok = prompt[0]
    print("q05 decode steps", flush=True)
    for pos in range(20):
        nxt = gm.forward(tok, pos)
        lg = gm.logits().astype(np.float64)
        rl, rt = rm.step(tok, pos)
        scale = np.sqrt(np.mean(rl.astype(np.float64) ** 2))
        _, d8 = oracle.quantize_q8(rm.head_x)
        tol = 2e-3 * scale + 4 * float(d8.max()) * wmax
        assert np.abs(lg - rl).max() <= tol, pos
        top = np.sort(rl)[-2:]
        if top[1] - top[0] > 2 * tol:
            assert nxt == rt, pos
        for li in range(cfg["n_layer"]):
            k, v = gm.kv_cache(li, pos + 1)
            for got, ref in ((k[pos], rm.K[li][pos]), (v[pos], rm.V[li][pos])):
                g, r = f16(got), f16(ref)
                ulp = np.abs(np.spacing(np.asarray(ref, np.uint16).view(np.float16))).astype(np.float64)
                rms = np.sqrt(np.mean(r ** 2))
                rel = 2e-4 if li == 0 else 1e-2
                assert np.all(np.abs(g - r) <= ulp + rel * rms), (pos, li)
        tok = prompt[pos + 1] if pos + 1 < len(prompt) else rt
    # the graph path (device-resident state) gives the eager tokens
    toks = gm.generate(prompt, 6)
    gm2 = DecodeModel.from_gguf(path, max_seq)
    toks2 = gm2.generate(prompt, 6, use_graph=False)
    assert list(toks) == list(toks2)
    gm.close()
    gm2.close()
