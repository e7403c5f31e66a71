"""The decode step reads K/V cache rows only below the position it decodes:
rows at and past that position hold whatever the allocation held (the
runtime does not clear the cache; the step writes row `pos` itself).  Those
rows are filled with NaN bit patterns in one model and with zeros in an
identical one, and the step's logits must be bit-identical.  Covers the
short-context attention (3B widths, 512-token context) and the long-context
matrix-core attention (7B widths, 2200-token context), on the multi-launch
path (3) and the persistent path (4)."""
import ctypes as C

import numpy as np
import pytest
import torch

from taraference_amd import synth

pytestmark = pytest.mark.gpu

CASES = {
    "3b_ctx512": (dict(n_layer=2, n_embd=2048, n_ff=11008, n_head=16, n_kv=2, head_dim=128,
                       n_vocab=3000, rope_theta=1e6, rms_eps=1e-6), 512),
    "7b_ctx2200": (dict(n_layer=2, n_embd=3584, n_ff=18944, n_head=28, n_kv=4, head_dim=128,
                        n_vocab=3000, rope_theta=1e6, rms_eps=1e-6), 2200),
}

_hip = None


def _memset(ptr, byte, n):
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so.7")
        _hip.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        _hip.hipMemset.restype = C.c_int
    assert _hip.hipMemset(C.c_void_p(ptr), byte, n) == 0


def _step(cfg, ctx, path, fill, seed):
    from taraference_amd.model import DecodeModel

    rng = np.random.default_rng(seed)
    layers = [synth.qwen_layer(rng, cfg, li, True) for li in range(cfg["n_layer"])]
    emb = synth.qwen_embedding(rng, cfg, True)
    max_seq = ctx + 4
    gm = DecodeModel(dict(cfg, max_seq=max_seq), layers, emb)
    gm.set_path(path)
    prompt = np.random.default_rng(seed + 1).integers(0, cfg["n_vocab"], ctx).tolist()
    tok = gm.prefill(prompt, 0)
    torch.cuda.synchronize()
    row = cfg["n_kv"] * cfg["head_dim"] * 2
    for li in range(cfg["n_layer"]):
        for get in (gm.lib.tf_model_k_cache, gm.lib.tf_model_v_cache):
            _memset(get(gm.h, li) + ctx * row, fill, (max_seq - ctx) * row)
    torch.cuda.synchronize()
    nxt = gm.forward(tok, ctx)
    lg = gm.logits()
    gm.close()
    return nxt, lg


@pytest.mark.parametrize("path", [3, 4])
@pytest.mark.parametrize("case", list(CASES))
def test_rows_past_position_do_not_matter(gpu, case, path):
    cfg, ctx = CASES[case]
    print(f"[cache-garbage] {case} path {path}: NaN-filled rows", flush=True)
    t_nan, l_nan = _step(cfg, ctx, path, 0xFF, 901)
    print(f"[cache-garbage] {case} path {path}: zero-filled rows", flush=True)
    t_zero, l_zero = _step(cfg, ctx, path, 0x00, 901)
    assert np.all(np.isfinite(l_nan))
    assert t_nan == t_zero
    assert np.array_equal(l_nan.view(np.uint32), l_zero.view(np.uint32))
