"""Pins for the oracle's decode-step glue: f16 conversions, RMSNorm, RoPE,
embedding-row dequantization and argmax (oracle/oracle.c).

Each is checked against something the oracle does not share code with:
numpy's IEEE half type, the reference's own f16 known answers
(crates/core/src/quant.rs:105-150), closed forms and invariants, and the
independent numpy dequantizers of tests/_util.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from taraference_amd import synth

from _util import matrix_blocks, q4k_dequant, q6k_dequant


# ------------------------------------------------------------------ f16

def test_f16_to_f32_all_patterns():
    """Every one of the 65536 half patterns decodes as IEEE binary16 does
    (kernels/common.cu:2-6 cvt.f32.f16)."""
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("v", [0.0, 1.0, -1.0, 0.5, 2.0, 65504.0, -0.25])
def test_f16_reference_known_answers(v):
    """The reference's f16_roundtrip_common_values (quant.rs:120-131): these
    values survive f32 -> f16 -> f32 (they are exact halves, so exactly)."""
    h = oracle.f32_to_f16_halfup(v)
    assert oracle.f16_to_f32(h) == v
    assert h == int(np.float16(v).view(np.uint16))


def test_f16_inf_nan():
    """quant.rs:133-139, and float_to_half_bits' overflow rule (common.cu:21-22)."""
    assert oracle.f32_to_f16_halfup(float("inf")) == 0x7C00
    assert oracle.f32_to_f16_halfup(float("-inf")) == 0xFC00
    assert (oracle.f32_to_f16_halfup(float("nan")) & 0x7C00) == 0x7C00
    assert oracle.f32_to_f16_halfup(65520.0) == 0x7C00     # halfway above max: up
    assert oracle.f32_to_f16_halfup(1e6) == 0x7C00


def test_f32_to_f16_is_nearest_with_ties_up():
    """float_to_half_bits (common.cu:9-38) adds the first dropped bit: the
    result is the nearest half, and exact ties go away from zero.  numpy's
    conversion is nearest-even, so the two agree except at ties, where ours
    is the one of larger magnitude."""
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(100),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),   # subnormal halves
        np.float32(2.0) ** rng.integers(-24, 15, 20000).astype(np.float32),
    ])
    got = oracle.f32_to_f16(x)
    rne = x.astype(np.float16).view(np.uint16)
    diff = got != rne
    # differences only at exact ties (value halfway between two halves)
    lo = got.view(np.float16).astype(np.float64)
    alt = rne.view(np.float16).astype(np.float64)
    xd = x.astype(np.float64)
    assert np.all(np.abs(np.abs(lo[diff] - xd[diff]) - np.abs(alt[diff] - xd[diff])) == 0)
    assert np.all(np.abs(lo[diff]) > np.abs(alt[diff]))
    # constructed ties: 1 + (2k+1) * 2^-11 lies halfway between two halves
    k = np.arange(0, 1024, dtype=np.float32)
    ties = np.float32(1.0) + (np.float32(2.0) * k + 1) * np.float32(2.0 ** -11)
    up = oracle.f32_to_f16(ties).view(np.float16).astype(np.float64)
    assert np.all(up > ties.astype(np.float64))


# ------------------------------------------------------------------ RMSNorm

def test_rms_norm_closed_form_and_f64():
    """ops.cu:4-34.  A constant row c with unit weights normalizes to
    c / sqrt(c^2 + eps); a random row matches the float64 formula to f32
    rounding."""
    n = 2048
    c = np.float32(0.75)
    out = oracle.rms_norm(np.full(n, c, np.float32), np.ones(n, np.float32), 1e-6)
    want = 0.75 / np.sqrt(0.75 ** 2 + 1e-6)
    assert np.allclose(out, want, rtol=2e-7)
    rng = np.random.default_rng(1)
    for n in (896, 2048, 3584):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        out = oracle.rms_norm(x, w, 1e-6).astype(np.float64)
        xd = x.astype(np.float64)
        ref = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w
        assert np.max(np.abs(out - ref) / np.abs(ref).clip(1e-3)) < 2e-6


def test_rms_norm_summation_order():
    """The sum of squares is formed in the reference's order: 256 strided
    per-thread sums, then a halving tree.  x[0] = 4096 (square 2^24) and
    ones on threads 1..255: the tree first pairs the ones (1+1 = 2, ...) and
    adds them to 2^24 as 2+4+...+128, so the sum is exactly 2^24 + 254; a
    sequential sum would lose every 1 against 2^24."""
    n = 512
    x = np.zeros(n, np.float32)
    x[0] = np.float32(4096.0)
    x[1:256] = np.float32(1.0)
    out = oracle.rms_norm(x, np.ones(n, np.float32), 0.0)
    s = np.float32(2.0 ** 24 + 254)
    scale = np.float32(1.0) / np.sqrt(s / np.float32(n))
    assert out[0] == np.float32(4096.0) * scale
    seq = np.float32(1.0) / np.sqrt(np.float32(2.0 ** 24) / np.float32(n))
    assert out[0] != np.float32(4096.0) * seq


# ------------------------------------------------------------------ RoPE

def test_rope_identity_and_rotation():
    """ops.cu:348-398 (NeoX pairs (i, i+hd/2), freq = theta^(-2i/hd)).
    pos 0 is the identity; pair norms are kept; angles match float64."""
    rng = np.random.default_rng(2)
    hd, nh, theta = 128, 4, 1e6
    x = rng.standard_normal(nh * hd).astype(np.float32)
    assert np.array_equal(oracle.rope_neox(x, nh, hd, 0, theta), x)
    pos = 37
    y = oracle.rope_neox(x, nh, hd, pos, theta).astype(np.float64).reshape(nh, hd)
    xd = x.astype(np.float64).reshape(nh, hd)
    i = np.arange(hd // 2)
    ang = pos * theta ** (-2.0 * i / hd)
    c, s = np.cos(ang), np.sin(ang)
    ref0 = xd[:, :hd // 2] * c - xd[:, hd // 2:] * s
    ref1 = xd[:, :hd // 2] * s + xd[:, hd // 2:] * c
    assert np.max(np.abs(y[:, :hd // 2] - ref0)) < 5e-5
    assert np.max(np.abs(y[:, hd // 2:] - ref1)) < 5e-5
    n0 = xd[:, :hd // 2] ** 2 + xd[:, hd // 2:] ** 2
    n1 = y[:, :hd // 2] ** 2 + y[:, hd // 2:] ** 2
    assert np.max(np.abs(n0 - n1) / n0.clip(1e-6)) < 1e-5


# ------------------------------------------------------------------ embedding

@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_embed_row_matches_numpy_dequant(kind):
    """embed.cu:51-131: row `token` of a K-quant table dequantized."""
    rng = np.random.default_rng(3)
    n_rows, n_vocab = 512, 20
    if kind == "q4k":
        w, cb = synth.q4k_matrix(rng, n_rows, n_vocab)
        bb, deq = 144, q4k_dequant
    else:
        w, cb = synth.q6k_matrix(rng, n_rows, n_vocab)
        bb, deq = 210, q6k_dequant
    for tok in (0, 7, n_vocab - 1):
        got = oracle.embed_row(w, bb, tok, n_rows, cb).astype(np.float64)
        want = deq(matrix_blocks(w, n_rows, bb)[tok]).reshape(-1)
        assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))


# ------------------------------------------------------------------ argmax

def _argmax_sim(x, threads=256):
    """Brute-force simulation of argmax_f32 (kernels/ops.cu:573-599) as one
    block of `threads` threads: each thread's strided strict-> scan from
    -1e30, then the halving tree in which slot t takes slot t+s only when
    strictly greater (Python floats; the comparisons are the same in fp32)."""
    slots = []
    for t in range(threads):
        bv, bi = -1e30, 0
        for i in range(t, len(x), threads):
            v = float(x[i])
            if v > bv:
                bv, bi = v, i
        slots.append((bv, bi))

    n = threads
    cur = list(slots)
    s = n // 2
    while s > 0:
        nxt = list(cur)
        for t in range(s):
            if cur[t + s][0] > cur[t][0]:
                nxt[t] = cur[t + s]
        cur = nxt
        s //= 2
    return cur[0][1]


def _argmax_rule(x):
    """The closed-form winner: among finite-or-inf values above -1e30 with
    the maximal value, the smallest 8-bit bit-reversed residue i mod 256,
    then the smallest i; index 0 when no value beats -1e30."""
    x = np.asarray(x, np.float32)
    ok = np.where(x > np.float32(-1e30))[0]
    if ok.size == 0:
        return 0
    m = x[ok].max()
    cand = ok[x[ok] == m]
    rev = [int(f"{int(i) & 255:08b}"[::-1], 2) for i in cand]
    return int(min(zip(rev, cand.tolist()))[1])


def test_argmax_reference_tie_rule_small():
    # hand cases from the tree's tie order
    for ties, want in (((1, 2), 2), ((10, 260), 260), ((64, 128), 128), ((0, 128), 0),
                       ((3, 259), 3), ((5, 7), 5), ((255, 511), 255), ((6, 1), 6)):
        x = np.zeros(600, np.float32) - 1
        for i in ties:
            x[i] = 7.0
        assert _argmax_sim(x) == want, ties
        assert oracle.argmax(x) == want, ties
        assert _argmax_rule(x) == want, ties


def test_argmax_reference_edges():
    # nothing above -1e30 -> 0; NaN and -inf never win; -0 ties with +0
    assert oracle.argmax(np.full(1000, -3e30, np.float32)) == 0
    assert oracle.argmax(np.full(1000, -1e30, np.float32)) == 0
    x = np.full(1000, np.nan, np.float32)
    x[700] = -5.0
    assert oracle.argmax(x) == 700
    x = np.full(1000, -np.inf, np.float32)
    assert oracle.argmax(x) == 0
    x = np.full(300, -1.0, np.float32)
    x[1], x[2] = np.float32(-0.0), np.float32(0.0)
    assert oracle.argmax(x) == _argmax_sim(x) == 2
    x[1], x[2] = np.float32(0.0), np.float32(-0.0)
    assert oracle.argmax(x) == 2
    x = np.full(10, -2.0, np.float32)
    x[9] = np.inf
    assert oracle.argmax(x) == 9
    assert oracle.argmax(np.array([3.0], np.float32)) == 0


@pytest.mark.parametrize("seed", range(6))
def test_argmax_against_simulation(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 3000))
    # few distinct values so ties across residues are common
    x = rng.integers(-4, 4, n).astype(np.float32)
    if seed % 2:
        x[rng.integers(0, n, n // 7)] = np.nan
    if seed == 5:
        x[:] = -1e31
        x[rng.integers(0, n, 3)] = -1e30
    want = _argmax_sim(x)
    assert oracle.argmax(x) == want
    assert _argmax_rule(x) == want


def test_argmax_vocab_random():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(151936).astype(np.float32)
    assert oracle.argmax(x) == int(np.argmax(x))  # distinct values: the plain argmax
    x[100] = x[90000] = np.float32(50.0)  # residues 100 (rev 38) and 144 (rev 9)
    assert oracle.argmax(x) == 90000 == _argmax_rule(x)
