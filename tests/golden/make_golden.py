"""Writes the golden fixtures of this directory from the CPU oracle.

The reference holds no vectors for its kernels (its tests pin only f16
conversion, registry names and tuning selection), so these fixtures are the
oracle's outputs on seeded synthetic inputs at the reference's shapes,
frozen: tests/test_golden.py checks that the oracle still reproduces them
(CPU) and that the HIP library matches them to the parity bar (GPU).

    python tests/golden/make_golden.py      # rewrites *.npz here

Inputs follow the synthetic distributions of the benchmark configs
(seed 0x7A7A0000 + config).  Weights are kept small (few columns) so the
files stay small; the column length K is the real one.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from taraference_amd import synth  # noqa: E402


def save(name, **arrays):
    np.savez_compressed(HERE / f"{name}.npz", **arrays)
    print(f"{name}.npz: " + ", ".join(f"{k}{list(v.shape)}" for k, v in arrays.items()))


def main():
    # Q8 activation quantize at configs 0, 1 and 4 widths (gemv.cu:43-65)
    for k, cfg in ((896, 0), (2048, 1), (3584, 4), (11008, 1)):
        rng = np.random.default_rng(0x7A7A0000 + cfg)
        x = synth.activation(rng, k)
        x[:32] = 0.0                       # an all-zero group
        x[32:64] *= np.float32(1e-30)      # a tiny-scale group
        q8, d8 = oracle.quantize_q8(x)
        save(f"q8_k{k}", x=x, q8=q8, d8=d8)

    # config 0: Q4_K x Q8, K = 896 (3 whole super-blocks), first 48 columns
    rng = np.random.default_rng(0x7A7A0000)
    w, cb = synth.q4k_matrix(rng, 896, 48)
    x = synth.activation(rng, 896)
    xq, xd = oracle.quantize_q8(x)
    y = oracle.gemv_q4k_q8(w, xq, xd, 896, 48, cb)
    y64, rowabs = oracle.gemv_q4k_q8_f64(w, xq, xd, 896, 48, cb)
    save("gemv_q4k_k896", w=w, col_bytes=np.int32(cb), xq=xq, xd=xd, y=y, y64=y64,
         rowabs=rowabs)

    # config 1a: fused gate+up, K = 2048, 32 columns
    rng = np.random.default_rng(0x7A7A0001)
    g, cb = synth.q4k_matrix(rng, 2048, 32)
    u, _ = synth.q4k_matrix(rng, 2048, 32)
    x = synth.activation(rng, 2048)
    xq, xd = oracle.quantize_q8(x)
    h = oracle.gemv_q4k_ffn(g, u, xq, xd, 2048, 32, cb)
    g64, ga = oracle.gemv_q4k_q8_f64(g, xq, xd, 2048, 32, cb)
    u64, ua = oracle.gemv_q4k_q8_f64(u, xq, xd, 2048, 32, cb)
    save("ffn_q4k_k2048", gate=g, up=u, col_bytes=np.int32(cb), xq=xq, xd=xd, h=h, g64=g64,
         ga=ga, u64=u64, ua=ua)

    # config 1b: compact Q6_K down, K = 11008 (43 super-blocks), 16 columns,
    # residual added in place
    rng = np.random.default_rng(0x7A7A0002)
    raw, _ = synth.q6k_matrix(rng, 11008, 16)
    comp, ccb = synth.q6k_compact(raw, 11008)
    x = synth.activation(rng, 11008)
    xq, xd = oracle.quantize_q8(x)
    res = rng.standard_normal(16).astype(np.float32)
    y = oracle.gemv_q6k_compact_q8_kway(comp, xq, xd, 11008, 16, ccb, 8, use_res=2,
                                        out=res)
    y64, rowabs = oracle.gemv_q6k_q8_f64(comp, 212, xq, xd, 11008, 16, ccb)
    save("down_q6k_k11008", w=comp, col_bytes=np.int32(ccb), xq=xq, xd=xd, residual=res, y=y,
         y64=y64, rowabs=rowabs)

    # config 2: split-KV flash decode, 16 q / 2 kv heads x 128, L = 130 (ragged
    # 8-way split: chunks of 17, the last one 11)
    rng = np.random.default_rng(0x7A7A0003)
    L, nh, nkv, hd = 130, 16, 2, 128
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = synth.kv_cache(rng, L, nkv, hd)
    vc = synth.kv_cache(rng, L, nkv, hd)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    part = oracle.flash_partial(q, kc, vc, nh, nkv, hd, L - 1, 8, scale)
    out = oracle.flash_reduce(part, nh, hd, 8)
    out64 = oracle.attn_f64(q, kc, vc, nh, nkv, hd, L, scale)
    save("flash_L130", q=q, k=kc, v=vc, scale=np.float32(scale), out=out, out64=out64)


if __name__ == "__main__":
    main()
