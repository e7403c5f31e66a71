"""GPU argmax against the reference's tie rule (kernels/ops.cu:573-599, one
256-thread block as layer.rs:2248-2255 launches it), restated by
oracle.argmax and pinned on the CPU by a brute-force simulation of the
block (test_oracle_glue.py).

Ties are planted where the rule matters: across residues mod 256 whose
bit-reversed order differs from their plain order (indices 1 and 2: the
reference returns 2; 10 and 260: 260), with NaN, -inf and values <= -1e30,
at the lm_head width 151936.  The fused lm_head argmax paths see ties through
duplicated weight columns: two equal columns give bit-equal logits (checked
as a precondition), and the index must be the one the rule picks."""
import numpy as np
import pytest
import torch

import oracle
from taraference_amd import synth
from _gpu import P, S, call, dev, empty, host

pytestmark = pytest.mark.gpu

VOCAB = 151936


def _gpu_argmax(x):
    idx = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    call("tf_argmax", P(dev(x)), x.size, P(idx), S())
    return int(host(idx)[0])


@pytest.mark.parametrize("ties,want", [((1, 2), 2), ((10, 260), 260), ((64, 128), 128),
                                       ((0, 128), 0), ((5, 7), 5), ((100, 90000), 90000),
                                       ((151935, 3), 3), ((255, 151807), 255)])
def test_argmax_planted_ties(gpu, ties, want):
    rng = np.random.default_rng(sum(ties))
    x = rng.standard_normal(VOCAB).astype(np.float32)
    for i in ties:
        x[i] = np.float32(40.0)
    assert oracle.argmax(x) == want
    assert _gpu_argmax(x) == want


@pytest.mark.parametrize("case", ["nan", "neg_inf", "floor", "zeros", "small_ints", "short"])
def test_argmax_edges(gpu, case):
    rng = np.random.default_rng(3)
    if case == "nan":
        x = rng.standard_normal(VOCAB).astype(np.float32)
        x[rng.integers(0, VOCAB, 5000)] = np.nan
    elif case == "neg_inf":
        x = np.full(VOCAB, -np.inf, np.float32)
    elif case == "floor":  # nothing beats -1e30 but one value at it: index 0
        x = np.full(VOCAB, -2e30, np.float32)
        x[777] = -1e30
    elif case == "zeros":  # -0 ties with +0
        x = np.full(VOCAB, -1.0, np.float32)
        x[1], x[2], x[513] = np.float32(-0.0), np.float32(0.0), np.float32(-0.0)
    elif case == "small_ints":  # many exact ties
        x = rng.integers(-3, 3, VOCAB).astype(np.float32)
    else:
        x = rng.integers(0, 2, 37).astype(np.float32)
    assert _gpu_argmax(x) == oracle.argmax(x)


@pytest.mark.parametrize("entry", ["q8", "head"])
def test_fused_head_argmax_duplicated_columns(gpu, entry):
    n_rows = 2048
    rng = np.random.default_rng(11)
    raw, _ = synth.q6k_matrix(rng, n_rows, VOCAB)
    x = synth.activation(rng, n_rows)
    nw = np.ones(n_rows, np.float32)
    xb = oracle.rms_norm(x, nw, 1e-6) if entry == "head" else x
    q8, d8 = oracle.quantize_q8(xb)
    comp, ccb = synth.q6k_compact(raw, n_rows)
    y64, _ = oracle.gemv_q6k_q8_f64(comp, 212, q8, d8, n_rows, VOCAB, ccb)
    a = int(np.argmax(y64))
    # b beats a under the rule (residue 0 has the best priority) / loses (residue 255)
    for b in ((a // 256) * 256 + (256 if a % 256 == 0 else 0), (a // 256) * 256 + 255):
        if b >= VOCAB or b == a:
            b = 255 if b != 255 else 511
        raw2 = raw.copy()
        raw2[b] = raw2[a]
        comp2, _ = synth.q6k_compact(raw2, n_rows)
        logits = empty(VOCAB)
        key = torch.zeros(1024, dtype=torch.int64, device="cuda")  # TF_ARGMAX_SLOTS
        idx = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        if entry == "q8":
            call("tf_gemv_q6k_q8_argmax", P(dev(comp2)), P(dev(q8)), P(dev(d8)), P(logits),
                 n_rows, VOCAB, ccb, P(key), S())
        else:
            call("tf_gemv_q6k_head_argmax", P(dev(comp2)), P(dev(x)), P(dev(nw)), 1e-6, P(logits),
                 n_rows, VOCAB, ccb, P(key), S())
        call("tf_argmax_key_finalize", P(key), P(idx), S())
        lg = host(logits)
        assert lg[a].view(np.uint32) == lg[b].view(np.uint32)
        got = int(host(idx)[0])
        want = oracle.argmax(lg)
        assert want in (a, b)
        assert got == want, (a, b, got, want)


@pytest.mark.parametrize("path", [0, 3, 4])
def test_decode_step_argmax_tie(gpu, path):
    """The runtime's step (path 0: tf_argmax; path 3: the fused lm_head
    argmax; path 4: the persistent step's lm_head) with the lm_head's top
    column duplicated at an index of better and of worse tie priority."""
    from taraference_amd.model import DecodeModel

    cfg = dict(n_layer=2, n_embd=2048, n_ff=11008, n_head=16, n_kv=2, head_dim=128,
               n_vocab=VOCAB, rope_theta=1e6, rms_eps=1e-6)
    rng = np.random.default_rng(21)
    layers = [synth.qwen_layer(rng, cfg, li) for li in range(2)]
    emb = synth.qwen_embedding(rng, cfg)
    head = synth.q6k_matrix(rng, cfg["n_embd"], VOCAB)
    tok, pos = 17, 0

    def run(head_w):
        m = DecodeModel(dict(cfg, max_seq=8), layers, emb, output=(head_w, head[1]))
        m.set_path(path)
        nxt = m.forward(tok, pos)
        lg = m.logits()
        m.close()
        return nxt, lg

    nxt, lg = run(head[0])
    assert nxt == oracle.argmax(lg)
    a = nxt
    for b in ((a // 256) * 256 + (256 if a % 256 == 0 else 0), (a // 256) * 256 + 255):
        if b >= VOCAB or b == a:
            b = 255 if b != 255 else 511
        w2 = head[0].copy()
        w2[b] = w2[a]
        nxt2, lg2 = run(w2)
        assert lg2[a].view(np.uint32) == lg2[b].view(np.uint32)
        want = oracle.argmax(lg2)
        assert want in (a, b)
        assert nxt2 == want, (path, a, b, nxt2, want)
