"""A decoder loaded from a GGUF file (DecodeModel.from_gguf: the reader plus
the reference's tensor placement, cuda/load.rs:166-420) runs exactly the
model built from the same weights in memory: identical greedy tokens and
bit-identical logits, on the default path and on the reference-order path,
with the lm_head tied (no output.weight) or stored separately."""
import numpy as np
import pytest

import _gguf_write as W
from taraference_amd import synth

pytestmark = pytest.mark.gpu

CFGS = [
    dict(n_layer=2, n_embd=256, n_ff=512, n_head=2, n_kv=1, head_dim=128, n_vocab=300,
         rope_theta=1e6, rms_eps=1e-6),
    dict(n_layer=2, n_embd=2048, n_ff=11008, n_head=16, n_kv=2, head_dim=128, n_vocab=2000,
         rope_theta=1e6, rms_eps=1e-6),
]


@pytest.mark.parametrize("tied", [True, False])
@pytest.mark.parametrize("ci", [0, 1])
def test_gguf_model_matches_in_memory_model(gpu, tmp_path, ci, tied):
    from taraference_amd.model import DecodeModel

    cfg = CFGS[ci]
    print(f"gguf model case {ci} tied={tied}", flush=True)
    rng = np.random.default_rng(50 + ci)
    layers = [synth.qwen_layer(rng, cfg, li) for li in range(cfg["n_layer"])]
    emb = synth.qwen_embedding(rng, cfg)
    onorm = (1.0 + 0.1 * rng.standard_normal(cfg["n_embd"])).astype(np.float32)
    meta, tens = W.model_tensors(cfg, layers, emb, output=None if tied else emb,
                                 output_norm=onorm)
    path = tmp_path / "m.gguf"
    W.write(path, meta, tens)
    max_seq = 40
    ref = DecodeModel(dict(cfg, max_seq=max_seq), layers, emb, output_norm=onorm)
    got = DecodeModel.from_gguf(path, max_seq)
    assert got.cfg == dict(cfg, max_seq=max_seq, rope_theta=np.float32(cfg["rope_theta"]),
                           rms_eps=np.float32(cfg["rms_eps"]))
    prompt = np.random.default_rng(ci).integers(0, cfg["n_vocab"], 10).tolist()
    for path_id in (None, 0):
        if path_id is not None:
            ref.set_path(path_id)
            got.set_path(path_id)
        assert ref.path() == got.path()
        t_ref = ref.generate(prompt, 8)
        l_ref = ref.logits()
        t_got = got.generate(prompt, 8)
        l_got = got.logits()
        assert list(t_got) == list(t_ref)
        assert np.array_equal(l_got, l_ref)
    ref.close()
    got.close()
