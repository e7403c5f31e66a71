#!/usr/bin/env python3
"""Benchmark: batch-1 greedy decode of a random-init Qwen2.5-3B-shaped
Q4_K_M model on one MI355X (config 3 of the baseline), the roofline of its
dominant kernel (the persistent decode-step kernel, one launch per token),
the standalone config-1a Q4_K GEMV (fused gate+up) for the metric's GEMV
part, and the CPU-oracle baseline timed on this host.

Workload: --warmup W forced decode steps build the synthetic context
(W = 512 by default, the config's context), then --steps K greedy decode
steps are timed (K = 256 by default).  Each step is one full decode forward
(36 layers + lm_head + argmax) replayed from a captured HIP graph; the token
feeds back on the device and the K generated tokens are copied to the host
once at the end.  value = K / elapsed.

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
DECODE_KERNEL = "tf_decode_persistent_kernel<8,1,16,3> (whole decode step, one launch per token)"
# Its HBM bytes per launch: rocprofv3 FETCH_SIZE + WRITE_SIZE (KiB per
# dispatch) scaled by the same counters' reading on a 256 MiB device copy
# (FETCH_SIZE counts half of what a read moves here: factor 2.000; WRITE_SIZE
# factor 1.000); the counter runs are kept in profiles/.
DECODE_TRAFFIC = int((974391.3 * 2.0 + 19600.0 * 1.0) * 1024)
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
    from taraference_amd import synth
    from taraference_amd.model import DecodeModel

    rng = np.random.default_rng(seed)
    t0 = time.time()
    layers = (synth.qwen_layer(rng, cfg, li) for li in range(cfg["n_layer"]))
    emb = synth.qwen_embedding(rng, cfg)
    m = DecodeModel(dict(cfg, max_seq=max_seq), layers, emb)
    log(f"[bench] model built in {time.time() - t0:.1f}s")
    return m


def decode_throughput(m, cfg, warmup, steps, seed):
    import torch

    rng = np.random.default_rng(seed + 1)
    prompt = rng.integers(0, cfg["n_vocab"], max(1, warmup)).tolist()
    # untimed: the forced context (graph capture happens on the first call)
    first = m.generate(prompt, 1, pos0=0, use_graph=True)
    torch.cuda.synchronize()
    # timed: `steps` decode steps continuing from the greedy token; HIP events
    # on the stream the step graph is replayed on bracket the same region
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    toks = m.generate([int(first[0])], steps, pos0=len(prompt), use_graph=True)
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
    out = {"config": "4: Qwen2.5-7B-shape Q4_K_M, 32768-token context, 128 greedy tokens",
           "path": m.path(), "prefill_tokens": ctx, "prefill_s": round(t_pf, 3),
           "prefill_tok_s": round(ctx / t_pf, 1), "decode_tokens": n_gen,
           "decode_tok_s": round(n_gen / dt, 2), "ms_per_token": round(dt * 1e3 / n_gen, 3),
           "ms_per_token_events": round(e0.elapsed_time(e1) / n_gen, 3),
           "weight_bytes_per_token": synth.weight_bytes(cfg),
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
    dt, toks, dt_ev = decode_throughput(m, cfg, context, steps, 5)
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


def kernel_table(iters):
    from taraference_amd import benchkit as B

    rows = [
        ("cfg0_q4k_896x4864", lambda: B.case_q4k_gemv(896, 4864, 0, iters)),
        ("cfg1a_q4k_gate_up_2048x2x11008", lambda: B.case_q4k_ffn(2048, 11008, 1, iters, False)),
        ("cfg1b_q6k_down_11008x2048", lambda: B.case_q6k(11008, 2048, 2, iters)),
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
    out = {}
    for name, fn in rows:
        r = B.report(name, fn())
        out[name] = {"us": round(r["per_us"], 2), "us_b2b": round(r["b2b_us"], 2),
                     "MB": round(r["bytes"] / 1e6, 3), "GBs": round(r["gbs"], 1),
                     "frac_hbm": round(r["frac"], 4)}
        if "n_split" in r:
            out[name]["n_split"] = r["n_split"]
        if "flops" in r:
            out[name]["TFLOPs"] = round(r["flops"] / (r["b2b_us"] * 1e-6) / 1e12, 1)
        log(f"[bench] {name}: {out[name]}")
    return out


def cpu_baseline(cfg, budget_s=20.0):
    """The oracle's Q4_K/Q6_K x Q8 dequant-and-dot (the reference arithmetic
    restated in C) on the host cores, on a bounded sample of the decode step:
    the GEMVs of one even (Q4_K down) and one odd (Q6_K down) layer plus the
    lm_head, repeated while the budget lasts; tok/s is extrapolated to the 36
    layers.  Attention is not included (0.1% of the bytes at L = 512)."""
    import oracle
    from taraference_amd import synth

    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    threads = max(1, min(16, avail))
    rng = np.random.default_rng(99)
    e, f = cfg["n_embd"], cfg["n_ff"]
    nq, nkv = cfg["n_head"] * cfg["head_dim"], cfg["n_kv"] * cfg["head_dim"]
    x_e = synth.activation(rng, e)
    x_f = synth.activation(rng, f)
    qe, de = oracle.quantize_q8(x_e)
    qf, df = oracle.quantize_q8(x_f)
    wq, cb = synth.q4k_matrix(rng, e, nq + 2 * nkv)  # q, k (Q4_K) and v-sized rows
    wo, _ = synth.q4k_matrix(rng, nq, e)
    g, _ = synth.q4k_matrix(rng, e, f)
    u, _ = synth.q4k_matrix(rng, e, f)
    d4, fcb = synth.q4k_matrix(rng, f, e)
    d6raw, _ = synth.q6k_matrix(rng, f, e)
    d6, d6cb = synth.q6k_compact(d6raw, f)
    del d6raw
    head_raw, _ = synth.q6k_matrix(rng, e, cfg["n_vocab"])
    head, hcb = synth.q6k_compact(head_raw, e)
    del head_raw

    def layer_pair():
        for down_q6 in (False, True):
            oracle.gemv_q4k_q8_mt(wq, qe, de, e, nq + 2 * nkv, cb, threads)
            oracle.gemv_q4k_q8_mt(wo, qe, de, nq, e, cb, threads)
            oracle.gemv_q4k_ffn_mt(g, u, qe, de, e, f, cb, threads)
            if down_q6:
                oracle.gemv_q6k_compact_q8_kway_mt(d6, qf, df, f, e, d6cb, 8, threads)
            else:
                oracle.gemv_q4k_q8_mt(d4, qf, df, f, e, fcb, threads)

    def lm_head():
        oracle.gemv_q6k_compact_q8_kway_mt(head, qe, de, e, cfg["n_vocab"], hcb, 1, threads)

    layer_pair()  # warm caches / threads
    t_pairs, t_heads = [], []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(t_pairs) < 2:
        t0 = time.perf_counter()
        layer_pair()
        t_pairs.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        lm_head()
        t_heads.append(time.perf_counter() - t0)
        if len(t_pairs) >= 20:
            break
    per_token = (cfg["n_layer"] / 2) * float(np.median(t_pairs)) + float(np.median(t_heads))
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(1.0 / per_token, 4), "unit": "tok/s", "cores": threads,
            "kind": "port",
            "sample": (f"oracle Q4_K/Q6_K x Q8 GEMVs of 2 layers (one Q4_K-down, one Q6_K-down)"
                       f" + lm_head, {len(t_pairs)} reps, median, extrapolated to "
                       f"{cfg['n_layer']} layers; attention excluded; CPU: {model}")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=512)
    ap.add_argument("--kernel-iters", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--path", type=int, default=None,
                    help="decode kernel sequence (tf_model_set_path); default: the library's")
    ap.add_argument("--only-roofline", action="store_true",
                    help="run only the copy calibration and the roofline kernel (for counter runs)")
    ap.add_argument("--config4", action="store_true",
                    help="BASELINE config 4 instead: Qwen2.5-7B shape, 32768-token context "
                         "filled by prefill, then 128 timed greedy tokens")
    ap.add_argument("--q05", action="store_true",
                    help="instead: a Qwen2.5-0.5B-layout model (Q5_0/Q8_0 896-wide matrices, "
                         "path 0), 512-token context, 256 timed greedy tokens")
    ap.add_argument("--only-prefill", action="store_true",
                    help="only the runtime's 512-token prefill of the 3B-shape model")
    ap.add_argument("--only-kernels", action="store_true",
                    help="run only the per-kernel table (for kernel traces)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the decode path is single-GPU; "
              f"--gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)

    import torch

    from taraference_amd import capi, synth

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
        print(json.dumps(q05_decode(args.warmup, max(2, args.steps))), flush=True)
        return
    if args.only_kernels:
        print(json.dumps({"kernels": kernel_table(args.kernel_iters)}), flush=True)
        return
    if args.only_prefill:
        cfg = dict(synth.QWEN25_3B)
        m = build_model(cfg, 0x7A7A0003, 1024)
        print(json.dumps({"prefill": prefill_throughput(m, cfg, 512)}), flush=True)
        m.close()
        return
    cfg = dict(synth.QWEN25_3B)
    steps = max(2, args.steps)
    max_seq = args.warmup + steps + 8
    m = build_model(cfg, 0x7A7A0003, max_seq)
    if args.path is not None:
        m.set_path(args.path)
    log("[bench] decode ...")
    dt, toks, dt_ev = decode_throughput(m, cfg, args.warmup, steps, 3)
    tok_s = steps / dt
    log(f"[bench] decode: {steps} tokens in {dt * 1e3:.1f} ms -> {tok_s:.1f} tok/s")
    wbytes = synth.weight_bytes(cfg)
    path = m.path()
    pf = prefill_throughput(m, cfg, 512)
    log(f"[bench] prefill: {pf}")
    m.close()
    del m
    torch.cuda.empty_cache()

    # the dominant kernel: one launch per decode step; algorithmic bytes per
    # launch = the weights once plus the K/V cache the attention reads (mean
    # context of the timed steps); average launch duration = HIP events
    # around the timed region on the launch stream / steps
    ctx_mean = args.warmup + steps / 2.0
    kv_bytes = int(2 * cfg["n_layer"] * ctx_mean * cfg["n_kv"] * cfg["head_dim"] * 2)
    step_bytes = wbytes + kv_bytes
    us_step = dt_ev / steps * 1e6
    step_gbs = step_bytes / (us_step * 1e-6) / 1e9
    roof = {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(step_gbs / HBM_PEAK_GBS, 4),
            "traffic": DECODE_TRAFFIC if path == 4 else None,
            "kernel": DECODE_KERNEL if path == 4 else f"decode step, path {path} (several kernels)",
            "bytes_per_launch": step_bytes, "us_per_launch": round(us_step, 2)}
    r = kernel_roofline(args.kernel_iters)
    # average launch duration = event pair around a graph of back-to-back
    # launches on the kernel's stream / launches
    achieved = r["bytes"] / (r["b2b_us"] * 1e-6) / 1e9
    roof_gemv = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                 "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                 "traffic": ROOFLINE_TRAFFIC,
                 "kernel": ROOFLINE_KERNEL,
                 "bytes_per_launch": int(r["bytes"]), "us_per_launch": round(r["b2b_us"], 3),
                 "us_per_launch_single": round(r["per_us"], 3)}
    table = {} if args.no_kernels else kernel_table(args.kernel_iters)
    cpu = None if args.no_cpu else cpu_baseline(cfg, args.cpu_budget)

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k x q8 int8 dot, fp32 accumulate",
        "data": "synthetic (random-init Qwen2.5-3B-shape Q4_K_M weights, seeded)",
        "config": {"workload": "config 3: Qwen2.5-3B-shape Q4_K_M greedy decode, batch 1",
                   "context": args.warmup, "decode_tokens": steps,
                   "weight_bytes_per_token": wbytes,
                   "effective_weight_GBs": round(wbytes * tok_s / 1e9, 1),
                   "parallelism": "single GPU"},
        "roofline": roof,
        "roofline_q4k_gemv": roof_gemv,
        "cpu_baseline": cpu,
        "prefill": pf,
        "kernels": table,
        "greedy_tokens_head": [int(t) for t in toks[:8]],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
