"""Kernel timing for the batch-1 decode hot path (used by bench.py).

Every case allocates enough distinct copies of its weights (>= 1 GiB in
total) that cycling through them defeats the 256 MB Infinity Cache, so each
launch streams its weights from HBM.  Time is taken with HIP events on the
stream the kernels run on (torch's current stream, handed to the library):
  - per-launch: an event pair around each launch, averaged;
  - back-to-back: one event pair around a burst of launches.
Algorithmic bytes per launch follow the reference GGUF block sizes (Q4_K
144 B, Q6_K 210 B per 256 weights, even where the 212-byte compact copy is
read; Q8_0 34 B and Q5_0 22 B per 32 weights), plus the activation once and the output once (twice with an in-place
residual).
"""
from __future__ import annotations

import numpy as np
import torch

from . import capi, synth

HBM_PEAK = 8.0e12
ROTATE_BYTES = 1 << 30


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _copies(arr: np.ndarray, nbytes_each: int):
    n = max(2, -(-ROTATE_BYTES // max(nbytes_each, 1)))
    base = _dev(arr)
    return [base] + [base.clone() for _ in range(n - 1)]


def time_launches(launch, n_rot: int, iters: int, warmup: int = 3):
    """launch(i, stream) enqueues the kernel(s) on copy i % n_rot on `stream`.

    Returns (per-launch mean us, back-to-back mean us):
      - per-launch: an event pair around each eagerly launched kernel (this
        includes the host launch latency of a lone launch);
      - back-to-back: `iters` launches captured in one HIP graph, replayed
        between one event pair on the stream the graph runs on, / iters —
        the kernel's average launch duration with no host in the loop.
    """
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream
    for i in range(warmup):
        launch(i % n_rot, s)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        starts[i].record(stream)
        launch(i % n_rot, s)
        ends[i].record(stream)
    torch.cuda.synchronize()
    per = float(np.mean([a.elapsed_time(b) for a, b in zip(starts, ends)])) * 1e3
    cap = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        for i in range(iters):
            launch(i % n_rot, cap.cuda_stream)
    graph.replay()  # upload + warm
    torch.cuda.synchronize()
    b0 = torch.cuda.Event(enable_timing=True)
    b1 = torch.cuda.Event(enable_timing=True)
    b0.record(stream)
    graph.replay()
    b1.record(stream)
    torch.cuda.synchronize()
    b2b = b0.elapsed_time(b1) * 1e3 / iters
    del graph
    return per, b2b


def _q8(x):
    xq = torch.empty(x.numel(), dtype=torch.int8, device="cuda")
    xd = torch.empty(x.numel() // 32, dtype=torch.float32, device="cuda")
    capi.call("tf_quantize_q8", x.data_ptr(), xq.data_ptr(), xd.data_ptr(), x.numel(),
              capi.stream_ptr())
    return xq, xd


def case_q4k_gemv(n_rows, n_cols, seed, iters):
    rng = np.random.default_rng(seed)
    w, cb = synth.q4k_matrix(rng, n_rows, n_cols)
    ws = _copies(w, w.nbytes)
    x = _dev(synth.activation(rng, n_rows))
    xq, xd = _q8(x)
    out = torch.empty(n_cols, device="cuda")
    lib = capi.load()

    def launch(i, s):
        lib.tf_gemv_q4k_q8(ws[i].data_ptr(), xq.data_ptr(), xd.data_ptr(), out.data_ptr(),
                           n_rows, n_cols, cb, 0, None, 0, None, s)

    per, b2b = time_launches(launch, len(ws), iters)
    nb = n_rows // 256
    alg = n_cols * nb * 144 + n_rows + n_rows // 32 * 4 + 4 * n_cols
    return dict(per_us=per, b2b_us=b2b, bytes=alg)


def case_stream(n_bytes, iters, blocks_per_cu=2, depth=8, contiguous=1):
    """The streaming-read floor: tf_stream_read_probe over n_bytes per launch,
    rotating through >= 1 GiB of distinct buffers like the GEMV cases."""
    ws = _copies(np.zeros(n_bytes, np.uint8), n_bytes)
    sink = torch.empty(8 * 1024, dtype=torch.int32, device="cuda")
    lib = capi.load()

    def launch(i, s):
        lib.tf_stream_read_probe(ws[i].data_ptr(), n_bytes, sink.data_ptr(), blocks_per_cu,
                                 depth, contiguous, s)

    per, b2b = time_launches(launch, len(ws), iters)
    return dict(per_us=per, b2b_us=b2b, bytes=n_bytes)


def case_q4k_splitk(n_rows, n_cols, seed, iters, n_split=4):
    """The reference's tall Q4_K path (kernels/gemv.cu:1877 split-K partials
    + :2243 reduce, in-place residual): two launches per GEMV."""
    rng = np.random.default_rng(seed)
    w, cb = synth.q4k_matrix(rng, n_rows, n_cols)
    ws = _copies(w, w.nbytes)
    x = _dev(synth.activation(rng, n_rows))
    xq, xd = _q8(x)
    part = torch.empty(n_split * n_cols, device="cuda")
    out = torch.zeros(n_cols, device="cuda")
    lib = capi.load()

    def launch(i, s):
        lib.tf_gemv_q4k_q8_splitk(ws[i].data_ptr(), xq.data_ptr(), xd.data_ptr(),
                                  part.data_ptr(), n_rows, n_cols, cb, n_split, s)
        lib.tf_gemv_splitk_reduce(part.data_ptr(), out.data_ptr(), n_cols, n_split, 0, None, 2,
                                  None, s)

    per, b2b = time_launches(launch, len(ws), iters)
    alg = n_cols * (n_rows // 256) * 144 + n_rows + n_rows // 8 + 8 * n_cols
    return dict(per_us=per, b2b_us=b2b, bytes=alg)


def case_q4k_ffn(n_rows, n_cols, seed, iters, f32_x=True):
    rng = np.random.default_rng(seed)
    g, cb = synth.q4k_matrix(rng, n_rows, n_cols)
    u, _ = synth.q4k_matrix(rng, n_rows, n_cols)
    gs = _copies(g, 2 * g.nbytes)
    us = [_dev(u)] + [None] * 0
    us = [us[0]] + [us[0].clone() for _ in range(len(gs) - 1)]
    x = _dev(synth.activation(rng, n_rows))
    xq, xd = _q8(x)
    out = torch.empty(n_cols, device="cuda")
    lib = capi.load()
    if f32_x:
        def launch(i, s):
            lib.tf_gemv_q4k_ffn_f32(gs[i].data_ptr(), us[i].data_ptr(), x.data_ptr(),
                                    out.data_ptr(), n_rows, n_cols, cb, s)
        act = 4 * n_rows
    else:
        def launch(i, s):
            lib.tf_gemv_q4k_ffn(gs[i].data_ptr(), us[i].data_ptr(), xq.data_ptr(),
                                xd.data_ptr(), out.data_ptr(), n_rows, n_cols, cb, s)
        act = n_rows + n_rows // 8
    per, b2b = time_launches(launch, len(gs), iters)
    alg = 2 * n_cols * (n_rows // 256) * 144 + act + 4 * n_cols
    return dict(per_us=per, b2b_us=b2b, bytes=alg)


def case_q4k_qkv(n_rows, n_q, n_kv, seed, iters):
    rng = np.random.default_rng(seed)
    wq, cb = synth.q4k_matrix(rng, n_rows, n_q)
    wk, _ = synth.q4k_matrix(rng, n_rows, n_kv)
    wv, _ = synth.q4k_matrix(rng, n_rows, n_kv)
    total = wq.nbytes + wk.nbytes + wv.nbytes
    qs, ks, vs = _copies(wq, total), None, None
    ks = [_dev(wk)]
    ks += [ks[0].clone() for _ in range(len(qs) - 1)]
    vs = [_dev(wv)]
    vs += [vs[0].clone() for _ in range(len(qs) - 1)]
    x = _dev(synth.activation(rng, n_rows))
    xq, xd = _q8(x)
    q = torch.empty(n_q, device="cuda")
    k = torch.empty(n_kv, device="cuda")
    v = torch.empty(n_kv, device="cuda")
    bq = torch.zeros(n_q, device="cuda")
    bk = torch.zeros(n_kv, device="cuda")
    lib = capi.load()

    def launch(i, s):
        lib.tf_gemv_q4k_qkv(qs[i].data_ptr(), ks[i].data_ptr(), vs[i].data_ptr(),
                            xq.data_ptr(), xd.data_ptr(), q.data_ptr(), k.data_ptr(),
                            v.data_ptr(), n_rows, n_q, n_kv, n_kv, cb, 1, bq.data_ptr(),
                            bk.data_ptr(), bk.data_ptr(), s)

    per, b2b = time_launches(launch, len(qs), iters)
    n = n_q + 2 * n_kv
    alg = n * (n_rows // 256) * 144 + n_rows + n_rows // 8 + 4 * n + 4 * n
    return dict(per_us=per, b2b_us=b2b, bytes=alg)


def case_q6k(n_rows, n_cols, seed, iters, entry="tf_gemv_q6k_down_splitk", use_res=2):
    rng = np.random.default_rng(seed)
    raw, _ = synth.q6k_matrix(rng, n_rows, n_cols)
    comp, ccb = synth.q6k_compact(raw, n_rows)
    del raw
    ws = _copies(comp, comp.nbytes)
    x = _dev(synth.activation(rng, n_rows))
    xq, xd = _q8(x)
    out = torch.zeros(n_cols, device="cuda")
    fn = getattr(capi.load(), entry)

    def launch(i, s):
        fn(ws[i].data_ptr(), xq.data_ptr(), xd.data_ptr(), out.data_ptr(), n_rows, n_cols,
           ccb, 0, None, use_res, None, s)

    per, b2b = time_launches(launch, len(ws), iters)
    alg = n_cols * (n_rows // 256) * 210 + n_rows + n_rows // 8 + 4 * n_cols * (2 if use_res == 2 else 1)
    return dict(per_us=per, b2b_us=b2b, bytes=alg)


def case_block32(fmt, n_rows, n_cols, seed, iters, entry=None):
    """Q8_0 x Q8 (tf_gemv_q8_0_q8) or Q5_0 x f32 (tf_gemv_q5_0_f32)."""
    rng = np.random.default_rng(seed)
    mk = synth.q8_0_matrix if fmt == "q8_0" else synth.q5_0_matrix
    w, cb = mk(rng, n_rows, n_cols)
    ws = _copies(w, w.nbytes)
    x = _dev(synth.activation(rng, n_rows))
    xq, xd = _q8(x)
    out = torch.empty(n_cols, device="cuda")
    lib = capi.load()
    if fmt == "q8_0":
        def launch(i, s):
            lib.tf_gemv_q8_0_q8(ws[i].data_ptr(), xq.data_ptr(), xd.data_ptr(), out.data_ptr(),
                                n_rows, n_cols, cb, 0, None, 0, None, s)
        act = n_rows + n_rows // 8
    else:
        def launch(i, s):
            lib.tf_gemv_q5_0_f32(ws[i].data_ptr(), x.data_ptr(), out.data_ptr(), n_rows,
                                 n_cols, cb, 0, None, 0, None, s)
        act = 4 * n_rows
    per, b2b = time_launches(launch, len(ws), iters)
    return dict(per_us=per, b2b_us=b2b, bytes=n_cols * cb + act + 4 * n_cols)


def case_q5_0_qkv(n_rows, n_q, n_kv, seed, iters):
    rng = np.random.default_rng(seed)
    wq, cb = synth.q5_0_matrix(rng, n_rows, n_q)
    wk, _ = synth.q5_0_matrix(rng, n_rows, n_kv)
    wv, _ = synth.q5_0_matrix(rng, n_rows, n_kv)
    total = wq.nbytes + wk.nbytes + wv.nbytes
    qs = _copies(wq, total)
    ks = [_dev(wk)]
    ks += [ks[0].clone() for _ in range(len(qs) - 1)]
    vs = [_dev(wv)]
    vs += [vs[0].clone() for _ in range(len(qs) - 1)]
    x = _dev(synth.activation(rng, n_rows))
    q = torch.empty(n_q, device="cuda")
    k = torch.empty(n_kv, device="cuda")
    v = torch.empty(n_kv, device="cuda")
    bq = torch.zeros(n_q, device="cuda")
    bk = torch.zeros(n_kv, device="cuda")
    lib = capi.load()

    def launch(i, s):
        lib.tf_gemv_q5_0_qkv(qs[i].data_ptr(), ks[i].data_ptr(), vs[i].data_ptr(), x.data_ptr(),
                             q.data_ptr(), k.data_ptr(), v.data_ptr(), n_rows, n_q, n_kv, n_kv,
                             cb, 1, bq.data_ptr(), bk.data_ptr(), bk.data_ptr(), s)

    per, b2b = time_launches(launch, len(qs), iters)
    n = n_q + 2 * n_kv
    return dict(per_us=per, b2b_us=b2b, bytes=n * cb + 4 * n_rows + 8 * n)


def case_gemm(fmt, n_rows, n_cols, n_tok, seed, iters):
    """Prefill GEMM (tf_gemm_q4k_f32 / tf_gemm_q6k_f32), x f32 [n_tok][K]."""
    rng = np.random.default_rng(seed)
    w, cb = (synth.q4k_matrix if fmt == "q4k" else synth.q6k_matrix)(rng, n_rows, n_cols)
    ws = _copies(w, w.nbytes)
    x = _dev(rng.standard_normal((n_tok, n_rows)).astype(np.float32))
    out = torch.empty(n_tok * n_cols, device="cuda")
    fn = getattr(capi.load(), f"tf_gemm_{fmt}_f32")

    def launch(i, s):
        fn(ws[i].data_ptr(), x.data_ptr(), out.data_ptr(), n_rows, n_cols, cb, n_tok, s)

    per, b2b = time_launches(launch, len(ws), iters)
    nb = n_rows // 256
    return dict(per_us=per, b2b_us=b2b, bytes=w.nbytes + 4 * n_tok * (n_rows + n_cols),
                flops=2.0 * n_tok * nb * 256 * n_cols)


def case_attn_prefill(n_head, n_kv, hd, n_q, seed, iters):
    rng = np.random.default_rng(seed)
    Kc = synth.kv_cache(rng, n_q, n_kv, hd)
    Vc = synth.kv_cache(rng, n_q, n_kv, hd)
    k, v = _dev(Kc), _dev(Vc)
    q = _dev(rng.standard_normal(n_q * n_head * hd).astype(np.float32))
    out = torch.empty(n_q * n_head * hd, device="cuda")
    lib = capi.load()
    scale = float(np.float32(1 / np.sqrt(hd)))

    def launch(i, s):
        lib.tf_attn_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), n_head,
                            n_kv, hd, 0, n_q, scale, s)

    per, b2b = time_launches(launch, 1, iters)
    # causal: query i attends i + 1 keys; QK^T and PV are 2 flops per MAC each
    pairs = n_q * (n_q + 1) / 2
    return dict(per_us=per, b2b_us=b2b, bytes=Kc.nbytes + Vc.nbytes + 8 * n_q * n_head * hd,
                flops=4.0 * n_head * hd * pairs)


def case_flash(L, n_head, n_kv, hd, seed, iters, n_split=None):
    rng = np.random.default_rng(seed)
    Kc = synth.kv_cache(rng, L, n_kv, hd)
    Vc = synth.kv_cache(rng, L, n_kv, hd)
    kvb = Kc.nbytes + Vc.nbytes
    ks = _copies(Kc, kvb)
    vs = [_dev(Vc)]
    vs += [vs[0].clone() for _ in range(len(ks) - 1)]
    q = _dev(rng.standard_normal(n_head * hd).astype(np.float32))
    lib = capi.load()
    if n_split is None:
        n_split = lib.tf_flash_decode_n_split(n_kv, L)
    part = torch.empty(n_head * n_split * (2 + hd), device="cuda")
    out = torch.empty(n_head * hd, device="cuda")
    scale = float(np.float32(1 / np.sqrt(hd)))

    def launch(i, s):  # the tf_flash_decode entry: partials and their merge
        lib.tf_flash_decode(q.data_ptr(), ks[i].data_ptr(), vs[i].data_ptr(), part.data_ptr(),
                            None, out.data_ptr(), None, None, n_head, n_kv, hd, L - 1, None,
                            n_split, scale, s)

    per, b2b = time_launches(launch, len(ks), iters)
    alg = kvb + 4 * n_head * hd * 2
    return dict(per_us=per, b2b_us=b2b, bytes=alg, n_split=n_split)


def report(name, r):
    gbs = r["bytes"] / (r["per_us"] * 1e-6) / 1e9
    r.update(name=name, gbs=gbs, frac=gbs * 1e9 / HBM_PEAK)
    return r
