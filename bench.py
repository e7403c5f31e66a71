#!/usr/bin/env python3
"""Benchmark: batch-1 greedy decode of a random-init Qwen2.5-3B-shaped
Q4_K_M model on one MI355X (config 3 of the baseline), the roofline of its
dominant kernel (the persistent decode-step kernel, one launch per token),
the standalone config-1a Q4_K GEMV (fused gate+up) for the metric's GEMV
part, and the CPU-oracle baseline timed on this host.

Workload: 512 forced decode steps build the synthetic context (config 3's
context, untimed), --warmup W greedy steps run untimed from position 512
(W = 16 by default), then --steps K greedy decode steps are timed from that
same position (K = 256 by default).  Each step is one full decode forward
(36 layers + lm_head + argmax) replayed from a captured HIP graph; the token
feeds back on the device and the K generated tokens are copied to the host
once at the end.  value = K / elapsed.

Beside it the same JSON line carries, each as its own guarded leg: the
prefill rate, the per-kernel table (configs 0-2, a4, lm_head, prefill
kernels), config 4 (a Qwen2.5-7B-shape model at a 32768-token context,
128 timed greedy tokens, with its roofline) and the CPU-oracle baseline.

Prints one JSON line on stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

# The dominant kernel of the timed workload: the persistent decode step (one
# launch per token, 99% of the GPU time in the kernel trace).
DECODE_KERNEL = ("tf_decode_persistent_kernel<8,1,16,3,false,false> (whole decode step, one "
                 "launch per token)")
# Its HBM bytes per launch: rocprofv3 FETCH_SIZE + WRITE_SIZE (KiB per
# dispatch, timed dispatches of `bench.py --only-decode --steps 64 --warmup 4`)
# scaled by the same counters' reading on a 256 MiB device copy (FETCH_SIZE
# counts half of what a read moves here: factor 2.000; WRITE_SIZE factor
# 1.000); the counter runs are kept in profiles/.  The figure belongs to the
# kernel source it was measured on (DECODE_TRAFFIC_SRC, the first 16 hex
# digits of the SHA-256 of decode_persistent.hip + .hpp); a run on other
# source reports traffic null rather than a stale number.
DECODE_TRAFFIC = int((1013669.6 * 2.0 + 24008.8 * 1.0) * 1024)
DECODE_TRAFFIC_SRC = "b52ba0cdb9b34fd8"


def _decode_src_hash() -> str:
    import hashlib

    h = hashlib.sha256()
    for name in ("decode_persistent.hip", "decode_persistent.hpp"):
        h.update((ROOT / "taraference_amd" / "csrc" / name).read_bytes())
    return h.hexdigest()[:16]


# The standalone config-1a GEMV (the tf_gemv_q4k_ffn entry point), reported
# beside it for the metric's "Q4_K GEMV % of HBM peak" part.
ROOFLINE_KERNEL = "tf_q4k_pair_rows_kernel<8,1,0> (fused Q4_K gate+up+SiLU, 2048 -> 2x11008)"
# FETCH_SIZE 12426.5 KiB x 2.000 + WRITE_SIZE 86 KiB x 1.000
ROOFLINE_TRAFFIC = int((12426.5 * 2.0 + 86.0 * 1.0) * 1024)

METRIC = "batch-1 decode tok/s, Qwen2.5-3B-shape Q4_K_M; Q4_K GEMV % of HBM peak"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_model(cfg, seed, max_seq):
    """Random-init weights of the config's shape, drawn from the
    well-conditioned block distribution (synth.q4k_blocks_wc /
    q6k_blocks_wc), so the greedy tokens vary from step to step; the bytes
    per token are those of any Q4_K_M model of the shape."""
    from taraference_amd import synth
    from taraference_amd.model import DecodeModel

    rng = np.random.default_rng(seed)
    t0 = time.time()
    layers = (synth.qwen_layer(rng, cfg, li, wc=True) for li in range(cfg["n_layer"]))
    emb = synth.qwen_embedding(rng, cfg, wc=True)
    m = DecodeModel(dict(cfg, max_seq=max_seq), layers, emb)
    log(f"[bench] model built in {time.time() - t0:.1f}s")
    return m


def decode_throughput(m, cfg, context, warmup, steps, seed):
    """Config-3 decode: `context` forced tokens build the context (untimed,
    captures the step graph), `warmup` greedy steps from position `context`
    (untimed), then `steps` greedy steps timed from the same position
    (rewriting the same K/V rows).  Returns host seconds, the tokens and the
    HIP-event seconds on the stream the step graph replays on."""
    import torch

    rng = np.random.default_rng(seed + 1)
    prompt = rng.integers(0, cfg["n_vocab"], context).tolist()
    first = m.generate(prompt, 1, pos0=0, use_graph=True)
    if warmup:
        m.generate([int(first[0])], warmup, pos0=context, use_graph=True)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    toks = m.generate([int(first[0])], steps, pos0=context, use_graph=True)
    e1.record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return dt, toks, e0.elapsed_time(e1) * 1e-3


def config4(ctx=32768, n_gen=128):
    """Config 4: a random-init Qwen2.5-7B-shape Q4_K_M model, the context
    written by tf_model_prefill (timed once), then n_gen greedy decode steps
    timed as in decode_throughput (HIP events on the replay stream)."""
    import torch

    from taraference_amd import synth

    cfg = dict(synth.QWEN25_7B)
    m = build_model(cfg, 0x7A7A0004, ctx + n_gen + 8)
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, cfg["n_vocab"], ctx).tolist()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    first = m.prefill(prompt, 0)
    t_pf = time.perf_counter() - t0
    m.generate([first], 2, pos0=ctx, use_graph=True)  # graph capture, untimed
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    toks = m.generate([first], n_gen, pos0=ctx, use_graph=True)
    e1.record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_ev = e0.elapsed_time(e1) / n_gen
    wbytes = synth.weight_bytes(cfg)
    # attention reads pos + 1 K/V rows at positions ctx .. ctx + n_gen - 1
    kv = int(2 * cfg["n_layer"] * (ctx + (n_gen + 1) / 2.0) * cfg["n_kv"] * cfg["head_dim"] * 2)
    gbs = (wbytes + kv) / (ms_ev * 1e-3) / 1e9
    out = {"config": "4: Qwen2.5-7B-shape Q4_K_M, 32768-token context, 128 greedy tokens",
           "path": m.path(), "prefill_tokens": ctx, "prefill_s": round(t_pf, 3),
           "prefill_tok_s": round(ctx / t_pf, 1), "decode_tokens": n_gen,
           "decode_tok_s": round(n_gen / dt, 2), "ms_per_token": round(dt * 1e3 / n_gen, 3),
           "ms_per_token_events": round(ms_ev, 3),
           "weight_bytes_per_token": wbytes,
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "kernel": "tf_decode_persistent_kernel<16,1,16,5,true> long-context "
                                  "instantiation (one launch per token)",
                        "bytes_per_launch": wbytes + kv, "us_per_launch": round(ms_ev * 1e3, 2)},
           "greedy_tokens_head": [int(t) for t in toks[:8]]}
    m.close()
    return out


def q05_decode(context, steps):
    """Decode tok/s of a random-init Qwen2.5-0.5B-layout model: the 896-row
    matrices Q5_0 (q/k/o/gate/up) and Q8_0 (v, tied embedding), ffn_down
    Q4_K/Q6_K; the runtime's reference operator sequence (path 0) replayed
    from a HIP graph; timed as decode_throughput."""
    from taraference_amd import synth
    from taraference_amd.model import DecodeModel

    cfg = dict(synth.QWEN25_05B)
    rng = np.random.default_rng(0x7A7A0005)
    t0 = time.time()
    layers = [synth.qwen05_layer(rng, cfg, li) for li in range(cfg["n_layer"])]
    emb = synth.qwen05_embedding(rng, cfg)
    m = DecodeModel(dict(cfg, max_seq=context + steps + 8), layers, emb)
    log(f"[bench] 0.5B-layout model built in {time.time() - t0:.1f}s, path {m.path()}")
    dt, toks, dt_ev = decode_throughput(m, cfg, context, 0, steps, 5)
    wbytes = sum(int(v[0].nbytes) for L in layers for k, v in L.items()
                 if isinstance(v, tuple)) + int(emb[0].nbytes)
    out = {"model": "Qwen2.5-0.5B layout (Q5_0/Q8_0 896-wide, Q4_K/Q6_K down, Q8_0 tied "
                    "embedding)", "path": m.path(), "context": context, "decode_tokens": steps,
           "tok_s": round(steps / dt, 1), "ms_per_token_events": round(dt_ev * 1e3 / steps, 3),
           "weight_bytes_per_token": wbytes}
    m.close()
    return out


def prefill_throughput(m, cfg, n_tok, reps=3):
    """Prompt tokens/s of the runtime's batched prefill (tf_model_prefill:
    n_tok tokens from position 0, K/V written, last-token logits), median of
    reps after one warm-up; host-timed, the call blocks on its stream."""
    import torch

    rng = np.random.default_rng(5)
    toks = rng.integers(0, cfg["n_vocab"], n_tok).tolist()
    m.prefill(toks, 0)
    times = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        m.prefill(toks, 0)
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    return {"prompt_tokens": n_tok, "ms": round(dt * 1e3, 2), "tok_s": round(n_tok / dt, 1)}


def kernel_roofline(iters):
    """Config 1a: fused gate+up 2048 -> 2 x 11008 with the Q8 activation
    prepared by tf_quantize_q8 (the decode runtime's path)."""
    from taraference_amd import benchkit as B

    r = B.report("q4k_gate_up", B.case_q4k_ffn(2048, 11008, 1, iters, f32_x=False))
    return r


def copy_calibration(n_bytes=256 << 20, reps=3):
    """A plain device-to-device copy of known size, for scaling the
    FETCH_SIZE / WRITE_SIZE counters of the roofline kernel."""
    import torch

    a = torch.ones(n_bytes // 4, device="cuda")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    return n_bytes


def kernel_table(iters, only=None):
    """Per-kernel GPU table; `only` keeps the rows whose name contains it."""
    from taraference_amd import benchkit as B

    rows = [
        ("cfg0_q4k_896x4864", lambda: B.case_q4k_gemv(896, 4864, 0, iters)),
        ("cfg1a_q4k_gate_up_2048x2x11008", lambda: B.case_q4k_ffn(2048, 11008, 1, iters, False)),
        ("cfg1b_q6k_down_11008x2048", lambda: B.case_q6k(11008, 2048, 2, iters)),
        # the reference's Q4_K ffn_down (18 of 36 layers): split-K + reduce
        ("a4_q4k_down_splitk4_11008x2048", lambda: B.case_q4k_splitk(11008, 2048, 14, iters)),
        ("q4k_down_single_pass_11008x2048", lambda: B.case_q4k_gemv(11008, 2048, 14, iters)),
        ("cfg1c_q4k_qkv_2048x2560", lambda: B.case_q4k_qkv(2048, 2048, 256, 3, iters)),
        ("lm_head_q6k_2048x151936", lambda: B.case_q6k(2048, 151936, 6, max(10, iters // 4),
                                                       "tf_gemv_q6k_compact_q8", 0)),
        # Qwen2.5-0.5B Q4_K_M widths (K = 896 is not a multiple of 256)
        ("q8_0_lm_head_896x151936", lambda: B.case_block32("q8_0", 896, 151936, 8,
                                                           max(10, iters // 4))),
        ("q5_0_ffn_896x4864", lambda: B.case_block32("q5_0", 896, 4864, 9, iters)),
        ("q5_0_qkv_896x1152", lambda: B.case_q5_0_qkv(896, 896, 128, 10, iters)),
        # prefill (512-token prompt, Qwen2.5-3B shapes)
        ("prefill_gemm_q4k_2048x11008_T512", lambda: B.case_gemm("q4k", 2048, 11008, 512, 11,
                                                                 max(5, iters // 10))),
        ("prefill_gemm_q6k_11008x2048_T512", lambda: B.case_gemm("q6k", 11008, 2048, 512, 12,
                                                                 max(5, iters // 10))),
        ("prefill_attn_16x2x128_T512", lambda: B.case_attn_prefill(16, 2, 128, 512, 13,
                                                                   max(5, iters // 10))),
    ]
    for L in (512, 4096, 32768):
        rows.append((f"cfg2_flash_L{L}_split8", lambda L=L: B.case_flash(L, 16, 2, 128, 7, iters, 8)))
        rows.append((f"cfg2_flash_L{L}_auto", lambda L=L: B.case_flash(L, 16, 2, 128, 7, iters)))
    rows.append(("flash_L512_split1", lambda: B.case_flash(512, 16, 2, 128, 7, iters, 1)))
    out = {}
    for name, fn in rows:
        if only and only not in name:
            continue
        r = B.report(name, fn())
        out[name] = {"us": round(r["per_us"], 2), "us_b2b": round(r["b2b_us"], 2),
                     "MB": round(r["bytes"] / 1e6, 3), "GBs": round(r["gbs"], 1),
                     "frac_hbm": round(r["frac"], 4),
                     "frac_hbm_b2b": round(r["bytes"] / (r["b2b_us"] * 1e-6) / 8e12, 4)}
        if "n_split" in r:
            out[name]["n_split"] = r["n_split"]
        if "flops" in r:
            out[name]["TFLOPs"] = round(r["flops"] / (r["b2b_us"] * 1e-6) / 1e12, 1)
        log(f"[bench] {name}: {out[name]}")
    return out


FLOOR_SIZES = [("2.1MB", 2122416), ("3.0MB", 2972160), ("12.7MB", 12710592),
               ("18.5MB", 18522240), ("25.4MB", 25408768), ("255.9MB", 255863296)]


def floor_table(iters, sweep=False, only_bytes=None):
    """The streaming-read floor (tf_stream_read_probe) at the GEMVs' byte
    counts (or at only_bytes alone); sweep=True also tries the grid,
    load-depth and access-pattern variants."""
    from taraference_amd import benchkit as B

    configs = ([(2, 8, 1)] if not sweep else
               [(1, 8, 0), (2, 8, 0), (4, 8, 0), (1, 4, 1), (1, 8, 1), (2, 4, 1), (2, 8, 1),
                (4, 4, 1), (4, 8, 1)])
    out = {}
    sizes = FLOOR_SIZES if not only_bytes else [(f"{only_bytes / 1e6:.1f}MB", only_bytes)]
    for label, nb in sizes:
        nb = (nb + 15) // 16 * 16
        for bpc, depth, contig in configs:
            key = f"stream_{label}_wg{bpc}_d{depth}_{'contig' if contig else 'inter'}"
            r = B.report(key, B.case_stream(nb, iters if nb < (64 << 20) else max(10, iters // 4),
                                            bpc, depth, contig))
            out[key] = {"us": round(r["per_us"], 2), "us_b2b": round(r["b2b_us"], 2),
                        "MB": round(nb / 1e6, 3), "GBs": round(r["gbs"], 1),
                        "frac_hbm": round(r["frac"], 4),
                        "frac_hbm_b2b": round(nb / (r["b2b_us"] * 1e-6) / 8e12, 4)}
            log(f"[bench] {key}: {out[key]}")
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _cpu_threads():
    """Every core this process may run on (the affinity mask; on the GPU
    boxes that is the one-GPU share of the host)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _median_us(fn, reps, warm=2):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)) * 1e6


def cpu_kernel_table(threads_all, reps=20):
    """The oracle's (the reference arithmetic restated in C) Q4_K/Q6_K x Q8
    GEMVs and flash-decode partial at configs 0, 1a, 1b, 1c and 2 on the
    host cores, single-threaded and on `threads_all` threads with output
    columns (heads for attention) partitioned; median of `reps` runs after
    two warm-up runs; GB/s over the same algorithmic bytes as the GPU table."""
    import oracle
    from taraference_amd import synth

    rng = np.random.default_rng(98)
    rows = {}

    def q8(k):
        return oracle.quantize_q8(synth.activation(rng, k))

    def add(name, nbytes, fn):
        r = {}
        for label, th in (("1t", 1), ("mt", threads_all)):
            us = _median_us(lambda: fn(th), reps)
            r[f"us_{label}"] = round(us, 1)
            r[f"GBs_{label}"] = round(nbytes / (us * 1e-6) / 1e9, 2)
        r["MB"] = round(nbytes / 1e6, 3)
        rows[name] = r
        log(f"[bench] cpu {name}: {r}")

    xq, xd = q8(896)
    w0, cb0 = synth.q4k_matrix(rng, 896, 4864)
    add("cfg0_q4k_896x4864", 4864 * 3 * 144 + 896 + 112 + 4 * 4864,
        lambda th: oracle.gemv_q4k_q8_mt(w0, xq, xd, 896, 4864, cb0, th))
    xq, xd = q8(2048)
    g, cb = synth.q4k_matrix(rng, 2048, 11008)
    u, _ = synth.q4k_matrix(rng, 2048, 11008)
    add("cfg1a_q4k_gate_up_2048x2x11008", 2 * 11008 * 8 * 144 + 2048 + 256 + 4 * 11008,
        lambda th: oracle.gemv_q4k_ffn_mt(g, u, xq, xd, 2048, 11008, cb, th))
    del g, u
    wqkv, cb = synth.q4k_matrix(rng, 2048, 2560)
    add("cfg1c_q4k_qkv_2048x2560", 2560 * 8 * 144 + 2048 + 256 + 4 * 2560,
        lambda th: oracle.gemv_q4k_q8_mt(wqkv, xq, xd, 2048, 2560, cb, th))
    xq, xd = q8(11008)
    raw, _ = synth.q6k_matrix(rng, 11008, 2048)
    d6, ccb = synth.q6k_compact(raw, 11008)
    del raw
    add("cfg1b_q6k_down_11008x2048", 2048 * 43 * 210 + 11008 + 1376 + 8 * 2048,
        lambda th: oracle.gemv_q6k_compact_q8_kway_mt(d6, xq, xd, 11008, 2048, ccb, 8, th))
    del d6
    n_head, n_kv, hd = 16, 2, 128
    sc = float(np.float32(1 / np.sqrt(hd)))
    q = synth.activation(rng, n_head * hd)
    for L in (512, 4096, 32768):
        Kc = synth.kv_cache(rng, L, n_kv, hd)
        Vc = synth.kv_cache(rng, L, n_kv, hd)
        add(f"cfg2_flash_L{L}_split8", 2 * L * n_kv * hd * 2 + 8 * n_head * hd,
            lambda th, Kc=Kc, Vc=Vc, L=L: oracle.flash_reduce(
                oracle.flash_partial_mt(q, Kc, Vc, n_head, n_kv, hd, L - 1, 8, sc, th),
                n_head, hd, 8))
    return rows


def cpu_decode_step(cfg, threads, context=512, budget_s=12.0):
    """One full config-3 decode step of the oracle on `threads` host
    threads: for every one of the 36 layers the Q8 quantize, QKV, split-KV
    attention over `context` positions (K/V ~ N(0,1) f16), wo, fused gate+up
    and the Q4_K or Q6_K down, then the lm_head; distinct random weights per
    layer (1.93 GB, as the GPU streams).  Median over as many steps as fit
    the budget (at least 3)."""
    import oracle
    from taraference_amd import synth

    rng = np.random.default_rng(97)
    e, f, hd = cfg["n_embd"], cfg["n_ff"], cfg["head_dim"]
    nh, nkv = cfg["n_head"], cfg["n_kv"]
    nq, nk = nh * hd, nkv * hd
    layers = []
    for li in range(cfg["n_layer"]):
        L = {"qkv": synth.q4k_matrix(rng, e, nq + 2 * nk), "wo": synth.q4k_matrix(rng, nq, e),
             "g": synth.q4k_matrix(rng, e, f), "u": synth.q4k_matrix(rng, e, f)}
        if synth.down_is_q6k(li):
            raw, _ = synth.q6k_matrix(rng, f, e)
            L["d6"] = synth.q6k_compact(raw, f)
        else:
            L["d4"] = synth.q4k_matrix(rng, f, e)
        layers.append(L)
    raw, _ = synth.q6k_matrix(rng, e, cfg["n_vocab"])
    head, hcb = synth.q6k_compact(raw, e)
    del raw
    Kc = synth.kv_cache(rng, context, nkv, hd)
    Vc = synth.kv_cache(rng, context, nkv, hd)
    x0 = synth.activation(rng, e)
    sc = float(np.float32(1 / np.sqrt(hd)))

    def step():
        x = x0
        for L in layers:
            qe, de = oracle.quantize_q8(x)
            qkv = oracle.gemv_q4k_q8_mt(L["qkv"][0], qe, de, e, nq + 2 * nk, L["qkv"][1], threads)
            part = oracle.flash_partial_mt(qkv[:nq], Kc, Vc, nh, nkv, hd, context - 1, 8, sc,
                                           threads)
            att = oracle.flash_reduce(part, nh, hd, 8)
            qa, da = oracle.quantize_q8(att)
            x = x + oracle.gemv_q4k_q8_mt(L["wo"][0], qa, da, nq, e, L["wo"][1], threads)
            qe, de = oracle.quantize_q8(x)
            h = oracle.gemv_q4k_ffn_mt(L["g"][0], L["u"][0], qe, de, e, f, L["g"][1], threads)
            qh, dh = oracle.quantize_q8(h)
            if "d6" in L:
                y = oracle.gemv_q6k_compact_q8_kway_mt(L["d6"][0], qh, dh, f, e, L["d6"][1], 8,
                                                       threads)
            else:
                y = oracle.gemv_q4k_q8_mt(L["d4"][0], qh, dh, f, e, L["d4"][1], threads)
            x = (x + y * np.float32(1e-3)).astype(np.float32)
        qe, de = oracle.quantize_q8(x)
        lg = oracle.gemv_q6k_compact_q8_kway_mt(head, qe, de, e, cfg["n_vocab"], hcb, 1, threads)
        return oracle.argmax(lg)

    step()  # warm-up
    ts = []
    t_start = time.perf_counter()
    while len(ts) < 3 or (time.perf_counter() - t_start < budget_s and len(ts) < 20):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts)


def cpu_baseline(cfg, budget_s=12.0, kernel_reps=20):
    """The reference's arithmetic (the oracle) on this host: config 3's
    whole decode step on all usable cores (tok/s = the value), plus the
    per-kernel table at configs 0-2 single-threaded and on all cores."""
    threads = _cpu_threads()
    t_step, n = cpu_decode_step(cfg, threads, budget_s=budget_s)
    table = cpu_kernel_table(threads, kernel_reps)
    return {"value": round(1.0 / t_step, 3), "unit": "tok/s", "cores": threads,
            "hardware_concurrency": os.cpu_count(), "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": (f"oracle (reference arithmetic in C) config-3 decode step: all "
                       f"{cfg['n_layer']} layers (Q8 quantize, QKV, 8-split flash attention at "
                       f"context 512, wo, gate+up+SiLU, Q4_K/Q6_K down) + lm_head + argmax on "
                       f"{threads} threads, median of {n} steps; per-kernel table: median of "
                       f"{kernel_reps} runs, 1 thread and {threads} threads"),
            "step_ms": round(t_step * 1e3, 1),
            "kernels": table,
            "note": "baseline, not target"}


CONTEXT = 512  # config 3: a 512-token context, then the greedy decode steps


def _leg(name, fn):
    """Run an optional bench leg; a failure is recorded, not raised."""
    try:
        return fn()
    except Exception as exc:  # noqa: BLE001
        log(f"[bench] {name} failed: {exc!r}")
        return {"error": f"{type(exc).__name__}: {exc}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256,
                    help="timed greedy decode steps (config 3: 256)")
    ap.add_argument("--warmup", type=int, default=16,
                    help="untimed greedy decode steps before the timed ones (same positions)")
    ap.add_argument("--kernel-iters", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--no-config4", action="store_true",
                    help="skip the config-4 leg (7B shape, 32768-token context)")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--path", type=int, default=None,
                    help="decode kernel sequence (tf_model_set_path); default: the library's")
    ap.add_argument("--only-roofline", action="store_true",
                    help="run only the copy calibration and the roofline kernel (for counter runs)")
    ap.add_argument("--only-decode", action="store_true",
                    help="run only the config-3 decode leg (for kernel traces and counter runs)")
    ap.add_argument("--config4", action="store_true",
                    help="BASELINE config 4 instead: Qwen2.5-7B shape, 32768-token context "
                         "filled by prefill, then 128 timed greedy tokens")
    ap.add_argument("--q05", action="store_true",
                    help="instead: a Qwen2.5-0.5B-layout model (Q5_0/Q8_0 896-wide matrices, "
                         "path 0), 512-token context, 256 timed greedy tokens")
    ap.add_argument("--only-prefill", action="store_true",
                    help="only the runtime's 512-token prefill of the 3B-shape model")
    ap.add_argument("--kernel-filter", default=None,
                    help="with --only-kernels: rows whose name contains this text")
    ap.add_argument("--only-floor", action="store_true",
                    help="only the streaming-read floor (tf_stream_read_probe)")
    ap.add_argument("--floor-sweep", action="store_true",
                    help="with --only-floor: also the grid, depth and pattern variants")
    ap.add_argument("--floor-bytes", type=int, default=None,
                    help="with --only-floor: this one size only (for counter runs)")
    ap.add_argument("--only-kernels", action="store_true",
                    help="run only the per-kernel table (for kernel traces)")
    ap.add_argument("--only-cpu", action="store_true",
                    help="run only the CPU baseline (no GPU needed)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every GPU box here has one GPU, so the "
              f"decode path is built and measured single-GPU (--gpus {args.gpus} is not "
              f"supported)", file=sys.stderr)
        sys.exit(2)

    from taraference_amd import synth

    if args.only_cpu:
        print(json.dumps({"cpu_baseline": cpu_baseline(dict(synth.QWEN25_3B), args.cpu_budget)}),
              flush=True)
        return

    import torch

    from taraference_amd import capi

    capi.load()
    if args.only_roofline:
        # counter runs: the copy of known size, then the roofline kernel alone
        copy_calibration()
        r = kernel_roofline(args.kernel_iters)
        print(json.dumps({"kernel": ROOFLINE_KERNEL, "bytes": int(r["bytes"]),
                          "us_b2b": round(r["b2b_us"], 3), "us_single": round(r["per_us"], 3)}))
        return
    if args.config4:
        print(json.dumps(config4()), flush=True)
        return
    if args.q05:
        print(json.dumps(q05_decode(CONTEXT, max(2, args.steps))), flush=True)
        return
    if args.only_floor:
        print(json.dumps({"floor": floor_table(args.kernel_iters, args.floor_sweep,
                                               args.floor_bytes)}), flush=True)
        return
    if args.only_kernels:
        print(json.dumps({"kernels": kernel_table(args.kernel_iters, args.kernel_filter)}),
              flush=True)
        return
    if args.only_prefill:
        cfg = dict(synth.QWEN25_3B)
        m = build_model(cfg, 0x7A7A0003, 1024)
        print(json.dumps({"prefill": prefill_throughput(m, cfg, 512)}), flush=True)
        m.close()
        return
    cfg = dict(synth.QWEN25_3B)
    steps = max(2, args.steps)
    warmup = max(0, args.warmup)
    # the context, the warm-up steps and the timed steps (both from position
    # CONTEXT) and the 512-token prefill leg all fit
    max_seq = CONTEXT + max(steps, warmup) + 8
    m = build_model(cfg, 0x7A7A0003, max_seq)
    if args.path is not None:
        m.set_path(args.path)
    log("[bench] decode ...")
    dt, toks, dt_ev = decode_throughput(m, cfg, CONTEXT, warmup, steps, 3)
    tok_s = steps / dt
    log(f"[bench] decode: {steps} tokens in {dt * 1e3:.1f} ms -> {tok_s:.1f} tok/s "
        f"(events {dt_ev * 1e3:.1f} ms)")
    wbytes = synth.weight_bytes(cfg)
    path = m.path()
    pf = None if args.only_decode else _leg("prefill", lambda: prefill_throughput(m, cfg, 512))
    if pf is not None:
        log(f"[bench] prefill: {pf}")
    m.close()
    del m
    torch.cuda.empty_cache()

    # the dominant kernel: one launch per decode step; algorithmic bytes per
    # launch = the weights once plus the K/V cache the attention reads (mean
    # context of the timed steps: positions CONTEXT .. CONTEXT+steps-1 attend
    # over pos+1 rows); average launch duration = HIP events around the timed
    # region on the launch stream / steps
    ctx_mean = CONTEXT + (steps + 1) / 2.0
    kv_bytes = int(2 * cfg["n_layer"] * ctx_mean * cfg["n_kv"] * cfg["head_dim"] * 2)
    step_bytes = wbytes + kv_bytes
    us_step = dt_ev / steps * 1e6
    step_gbs = step_bytes / (us_step * 1e-6) / 1e9
    roof = {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(step_gbs / HBM_PEAK_GBS, 4),
            "traffic": (DECODE_TRAFFIC if path == 4 and _decode_src_hash() == DECODE_TRAFFIC_SRC
                        else None),
            "kernel": DECODE_KERNEL if path == 4 else f"decode step, path {path} (several kernels)",
            "bytes_per_launch": step_bytes, "us_per_launch": round(us_step, 2)}
    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(dt * 1e3 / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k x q8 int8 dot, fp32 accumulate",
        "data": "synthetic (random-init Qwen2.5-3B-shape Q4_K_M weights, seeded)",
        "config": {"workload": "config 3: Qwen2.5-3B-shape Q4_K_M greedy decode, batch 1, "
                               "512-token context",
                   "context": CONTEXT, "decode_tokens": steps, "decode_path": path,
                   "weight_bytes_per_token": wbytes,
                   "effective_weight_GBs": round(wbytes * tok_s / 1e9, 1),
                   "parallelism": "single GPU"},
        "roofline": roof,
    }
    if not args.only_decode:
        def gemv_roof():
            r = kernel_roofline(args.kernel_iters)
            # average launch duration = event pair around a graph of
            # back-to-back launches on the kernel's stream / launches
            achieved = r["bytes"] / (r["b2b_us"] * 1e-6) / 1e9
            return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": ROOFLINE_TRAFFIC, "kernel": ROOFLINE_KERNEL,
                    "bytes_per_launch": int(r["bytes"]), "us_per_launch": round(r["b2b_us"], 3),
                    "us_per_launch_single": round(r["per_us"], 3)}

        out["roofline_q4k_gemv"] = _leg("roofline_q4k_gemv", gemv_roof)
        out["prefill"] = pf
        out["kernels"] = {} if args.no_kernels else _leg("kernels",
                                                         lambda: kernel_table(args.kernel_iters))
        out["streaming_floor"] = {} if args.no_kernels else _leg(
            "streaming_floor", lambda: floor_table(args.kernel_iters))
        if not args.no_config4:
            log("[bench] config 4 ...")
            out["config4"] = _leg("config4", config4)
            log(f"[bench] config 4: {out['config4']}")
    out["cpu_baseline"] = (None if args.no_cpu or args.only_decode
                           else _leg("cpu_baseline", lambda: cpu_baseline(cfg, args.cpu_budget)))
    out["greedy_tokens_head"] = [int(t) for t in toks[:8]]
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
