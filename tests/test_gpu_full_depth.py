"""Full-depth decode parity: the real config-3 model (Qwen2.5-3B shape, 36
layers, vocab 151936) at a 512-token context and the config-4 model
(Qwen2.5-7B shape, 28 layers, vocab 152064) at a 4096-token context and at
its full 32768-token context, the
default persistent step (path 4) checked stage by stage, in every layer,
against the oracle's fp64 truths (the reference's op order: forward.rs:
360-407, layer.rs attn_block / ffn_block_dense).

Why stage by stage.  The step re-quantizes its activations to Q8 four
times per layer.  An fp32 summation-order difference of one ulp moves a
value across a Q8 rounding boundary now and then, and that one-step change
perturbs every output of the next GEMV enough to flip hundreds of roundings
further down.  Two correct implementations in different summation orders
therefore drift apart with depth: the CPU reference step itself, with one
ulp of noise added to each GEMV output, moves its own 36-layer logits by up
to 14% of their RMS on well-conditioned weights.  End-to-end logits cannot
be held to the fp32 tolerance at this depth; each stage, given its actual
input, can.

So the runtime keeps every layer's stage vectors (tf_model_keep_stage_vectors)
and a record of every quantizer's f32 input and Q8 output, and each stage is
fed the GPU's own input (teacher forcing):
  - every Q8 the step forms in-kernel (the QKV, gate/up and lm_head inputs
    after RMSNorm, the merged attention output, h) is checked byte for byte
    against quantize_q8_global (gemv.cu:43-65, the oracle) of the f32 values
    the kernel quantized, and the published Q8 against the recorded one;
  - the RMSNorm outputs within two f32 ulps of the oracle's;
  - QKV: the roped query and the new f16 K/V rows against fp64 GEMVs of the
    oracle's Q8 rotated by the reference's fp32 RoPE angles; 1e-5 of the
    GEMV terms plus the angle's fp32 rounding at that position, one f16 ulp
    for the cache rows;
  - attention over the GPU's K/V cache: the merged f32 output within 1e-4 of
    the fp64 softmax attention;
  - wo on the GPU's attention Q8, plus the residual: GEMV tolerance;
  - gate/up with SiLU: h within the GEMV tolerance propagated through SiLU;
  - down on the GPU's h Q8, plus the residual: GEMV tolerance;
  - the lm_head on the last residual: GEMV tolerance, and the token is the
    reference argmax of the GPU's logits (and the fp64 argmax when clear).
Then the production layout (two alternating stage buffers, no record) runs
the same step from the same prompt and must give bit-identical logits.

Two weight distributions: the benchmark's (scores of order
1e5, a near one-hot softmax) and a well-conditioned one (synth.q4k_blocks_wc
/ q6k_blocks_wc: activations, scores and logits of order 1)."""
import numpy as np
import pytest

import oracle
from taraference_amd import synth
from _util import GEMV_RTOL, CANCEL_FLOOR, gemv_tol

pytestmark = pytest.mark.gpu

ATT_TOL = 1e-4   # attention values (well inside the 2e-3 bar)


def _ulp32(x):
    return np.abs(np.spacing(np.asarray(x, np.float32))).astype(np.float64)


def _rope_cs(n, hd, pos, theta):
    """(cos, sin) per pair index as the reference's fp32 formula gives them
    (oracle.rope_neox on unit vectors), and a bound on the angle's error
    from fp32 rounding of freq and pos*freq."""
    e0 = np.zeros(hd, np.float32)
    cs = np.zeros((hd // 2, 2))
    for i in range(hd // 2):
        v = e0.copy()
        v[i] = 1
        r = oracle.rope_neox(v, 1, hd, pos, theta)
        cs[i] = r[i], r[i + hd // 2]
    i = np.arange(hd // 2)
    freq = theta ** (-2.0 * i / hd)
    dang = 2 * pos * freq * 2.0 ** -23 + 2 * _ulp32(pos * freq) + 1e-7
    return cs, dang


def _rope64(y, n_heads, hd, cs):
    y = y.reshape(n_heads, hd).astype(np.float64)
    h = hd // 2
    x0, x1 = y[:, :h], y[:, h:]
    c, s = cs[:, 0], cs[:, 1]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=1).reshape(-1)


def _rope_tol(y64, tol, n_heads, hd, dang):
    """Tolerance after the rotation: the pair's two GEMV tolerances plus
    |x| times the angle bound."""
    y = y64.reshape(n_heads, hd)
    t = tol.reshape(n_heads, hd)
    h = hd // 2
    mag = np.sqrt(y[:, :h] ** 2 + y[:, h:] ** 2)
    tp = t[:, :h] + t[:, h:] + mag * dang
    return np.concatenate([tp, tp], axis=1).reshape(-1)


def _check_close(got, ref, tol, what):
    err = np.abs(np.asarray(got, np.float64) - ref)
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, (f"{what}: {bad.size} values out of tolerance, worst i={bad[0]} "
                           f"err={err[bad].max():.3e} tol={tol[bad].min():.3e}")
    return float((err / np.maximum(tol, 1e-30)).max())


def _check_q8_exact(gm, site, li, what, published=None):
    """The Q8 the step's in-kernel quantizer produced at `site` of layer li
    equals, byte for byte, quantize_q8_global (kernels/gemv.cu:43-65, the
    oracle) of the f32 values that quantizer consumed; and, for the
    published vectors, what the next stage read is that Q8.  Returns the
    recorded f32 values."""
    x, q, d = gm.q8_record(site, li)
    q_ref, d_ref = oracle.quantize_q8(x)
    nq = int((q != q_ref).sum())
    assert nq == 0, f"{what}: {nq} Q8 values differ from quantize_q8 of the GPU's f32 input"
    assert np.array_equal(d.view(np.uint32), d_ref.view(np.uint32)), f"{what}: Q8 scales differ"
    if published is not None:
        pq, pd = published
        assert np.array_equal(pq, q) and np.array_equal(pd.view(np.uint32), d.view(np.uint32)), \
            f"{what}: the published Q8 is not the recorded one"
    return x


def _check_norm(x_gpu, ref, what):
    """RMSNorm output (x * scale * w in f32) against the oracle's: within two
    f32 ulps; returns the count of values that are not bit-identical."""
    x_gpu = np.asarray(x_gpu, np.float32)
    ref = np.asarray(ref, np.float32)
    err = np.abs(x_gpu.astype(np.float64) - ref)
    tol = 2 * _ulp32(ref) + 1e-38
    assert np.all(err <= tol), f"{what}: worst {err.max():.3e}"
    return int((x_gpu.view(np.uint32) != ref.view(np.uint32)).sum())


def _layers(cfg, wc, seed):
    """The model's layers, generated one at a time (seeded)."""
    rng = np.random.default_rng(seed)
    return (synth.qwen_layer(rng, cfg, li, wc) for li in range(cfg["n_layer"]))


def _run(cfg, context, wc, seed):
    from taraference_amd.model import DecodeModel

    c = cfg
    E, F, hd = c["n_embd"], c["n_ff"], c["head_dim"]
    H, KV = c["n_head"], c["n_kv"]
    nq, nk = H * hd, KV * hd
    layers = list(_layers(cfg, wc, seed))
    emb = synth.qwen_embedding(np.random.default_rng(seed + 2), cfg, wc)
    gm = DecodeModel(dict(cfg, max_seq=context + 2), layers, emb)
    assert gm.path() == 4
    gm.keep_stage_vectors(True)
    prompt = np.random.default_rng(seed + 1).integers(0, c["n_vocab"], context).tolist()
    tok = gm.prefill(prompt, 0)
    pos = context
    print(f"[full-depth] step pos={pos} tok={tok}", flush=True)
    nxt = gm.forward(tok, pos)
    logits = gm.logits()
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    cs, dang = _rope_cs(nq, hd, pos, c["rope_theta"])
    norm_diff = 0
    worst = {}
    x_in = oracle.embed_row(emb[0], 210, tok, E, emb[1])
    for li, L in enumerate(layers):
        # ---- QKV from the GPU's layer input
        xb = oracle.rms_norm(x_in, L["attn_norm"], c["rms_eps"])
        xb_gpu = _check_q8_exact(gm, gm.Q8_QKV_IN, li, f"layer {li} QKV input Q8")
        norm_diff += _check_norm(xb_gpu, xb, f"layer {li} attention RMSNorm")
        q8, d8 = oracle.quantize_q8(xb)
        cb = L["wq"][1]
        yq, aq = oracle.gemv_q4k_q8_f64(L["wq"][0], q8, d8, E, nq, cb)
        yk, ak = oracle.gemv_q4k_q8_f64(L["wk"][0], q8, d8, E, nk, cb)
        yv, av = oracle.gemv_q6k_f32_f64(L["wv"][0], xb, E, nk, L["wv"][1])
        yq, yk, yv = yq + L["bq"], yk + L["bk"], yv + L["bv"]
        q_ref = _rope64(yq, H, hd, cs)
        k_ref = _rope64(yk, KV, hd, cs)
        q_tol = _rope_tol(yq, gemv_tol(yq, aq), H, hd, dang)
        k_tol = _rope_tol(yk, gemv_tol(yk, ak), KV, hd, dang)
        q_gpu, _ = gm.stage_vector(gm.STAGE_Q, li)
        worst["q"] = max(worst.get("q", 0), _check_close(q_gpu, q_ref, q_tol + _ulp32(q_ref),
                                                         f"layer {li} roped q"))
        Kc, Vc = gm.kv_cache(li, pos + 1)
        k_row = Kc[pos].view(np.float16).astype(np.float64)
        v_row = Vc[pos].view(np.float16).astype(np.float64)
        f16ulp = lambda r: np.abs(np.spacing(r.astype(np.float16))).astype(np.float64)  # noqa
        _check_close(k_row, k_ref, k_tol + f16ulp(k_ref), f"layer {li} K row")
        _check_close(v_row, yv, gemv_tol(yv, av) + f16ulp(yv), f"layer {li} V row")
        # ---- attention over the GPU's cache with the GPU's query
        att = oracle.attn_f64(q_gpu, Kc, Vc, H, KV, hd, pos + 1, scale)
        (oq, od), _ = gm.stage_vector(gm.STAGE_O, li)
        att_gpu = _check_q8_exact(gm, gm.Q8_ATTN, li, f"layer {li} attention Q8", (oq, od))
        worst["att"] = max(worst.get("att", 0),
                           _check_close(att_gpu, att, np.full(att.size, ATT_TOL),
                                        f"layer {li} attention output"))
        # ---- wo + residual on the GPU's attention Q8
        yo, ao = oracle.gemv_q4k_q8_f64(L["wo"][0], oq, od, nq, E, L["wo"][1])
        xa_ref = x_in.astype(np.float64) + yo
        xa, _ = gm.stage_vector(gm.STAGE_XA, li)
        worst["wo"] = max(worst.get("wo", 0),
                          _check_close(xa, xa_ref, gemv_tol(yo, ao) + 2 * _ulp32(xa_ref),
                                       f"layer {li} residual after wo"))
        # ---- gate/up + SiLU from the GPU's residual
        xb2 = oracle.rms_norm(xa, L["ffn_norm"], c["rms_eps"])
        xb2_gpu = _check_q8_exact(gm, gm.Q8_GU_IN, li, f"layer {li} gate/up input Q8")
        norm_diff += _check_norm(xb2_gpu, xb2, f"layer {li} FFN RMSNorm")
        q8, d8 = oracle.quantize_q8(xb2)
        g64, ga = oracle.gemv_q4k_q8_f64(L["gate"][0], q8, d8, E, F, L["gate"][1])
        u64, ua = oracle.gemv_q4k_q8_f64(L["up"][0], q8, d8, E, F, L["up"][1])
        sig = np.exp(-np.logaddexp(0.0, -g64))  # 1 / (1 + e^-g) without overflow
        h_ref = g64 * sig * u64
        dsilu = sig * (1.0 + g64 * (1.0 - sig))
        h_tol = GEMV_RTOL * (np.abs(dsilu * u64) * np.maximum(np.abs(g64), CANCEL_FLOOR * ga)
                             + np.abs(g64 * sig) * np.maximum(np.abs(u64), CANCEL_FLOOR * ua)
                             + np.abs(h_ref)) + 1e-30
        (hq, hdq), _ = gm.stage_vector(gm.STAGE_H, li)
        h_gpu = _check_q8_exact(gm, gm.Q8_H, li, f"layer {li} h Q8", (hq, hdq))
        worst["h"] = max(worst.get("h", 0), _check_close(h_gpu, h_ref, h_tol, f"layer {li} h"))
        # ---- down + residual on the GPU's h Q8
        if L["down_q6k"]:
            comp, ccb = synth.q6k_compact(L["down"][0], F)
            yd, ad = oracle.gemv_q6k_q8_f64(comp, 212, hq, hdq, F, E, ccb)
        else:
            yd, ad = oracle.gemv_q4k_q8_f64(L["down"][0], hq, hdq, F, E, L["down"][1])
        xo_ref = xa.astype(np.float64) + yd
        xo, _ = gm.stage_vector(gm.STAGE_XB, li)
        worst["down"] = max(worst.get("down", 0),
                            _check_close(xo, xo_ref, gemv_tol(yd, ad) + 2 * _ulp32(xo_ref),
                                         f"layer {li} residual after down"))
        x_in = xo
    # ---- lm_head on the GPU's last residual
    xb = oracle.rms_norm(x_in, np.ones(E, np.float32), c["rms_eps"])
    xh_gpu = _check_q8_exact(gm, gm.Q8_QKV_IN, c["n_layer"], "lm_head input Q8")
    norm_diff += _check_norm(xh_gpu, xb, "output RMSNorm")
    q8, d8 = oracle.quantize_q8(xb)
    comp, ccb = synth.q6k_compact(emb[0], E)
    y64, ay = oracle.gemv_q6k_q8_f64(comp, 212, q8, d8, E, c["n_vocab"], ccb)
    worst["head"] = _check_close(logits, y64, gemv_tol(y64, ay), "logits")
    assert nxt == oracle.argmax(logits)
    srt = np.sort(y64)
    if srt[-1] - srt[-2] > 2 * gemv_tol(srt[-1:], ay.max(keepdims=True))[0]:
        assert nxt == int(np.argmax(y64))
    print(f"[full-depth] {c['n_layer']} layers: worst error/tolerance {worst}; "
          f"every Q8 bit-exact; {norm_diff} RMSNorm values not bit-identical to the oracle's",
          flush=True)
    gm.close()
    # The production layout (two alternating stage buffers, no record) runs
    # the same arithmetic at other addresses: the same token and logits.
    gm2 = DecodeModel(dict(cfg, max_seq=context + 2), _layers(cfg, wc, seed), emb)
    assert gm2.path() == 4
    assert gm2.prefill(prompt, 0) == tok
    assert gm2.forward(tok, pos) == nxt
    assert np.array_equal(gm2.logits().view(np.uint32), logits.view(np.uint32)), \
        "two-buffer step logits differ from the kept-vector step's"
    gm2.close()


@pytest.mark.parametrize("wc", [True, False], ids=["well_conditioned", "baseline_dist"])
def test_config3_full_depth(gpu, wc):
    _run(dict(synth.QWEN25_3B), 512, wc, 0x7A7A0003)


@pytest.mark.parametrize("wc", [True, False], ids=["well_conditioned", "baseline_dist"])
def test_config4_full_depth(gpu, wc):
    _run(dict(synth.QWEN25_7B), 4096, wc, 0x7A7A0004)


def test_config4_full_depth_full_context(gpu):
    """Config 4 jointly at full depth (28 layers) and full context (32768
    tokens written by the runtime's prefill), every stage of every layer
    checked as above."""
    _run(dict(synth.QWEN25_7B), 32768, True, 0x7A7A0014)
