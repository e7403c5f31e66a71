"""Shared test helpers: independent numpy dequantizers and tolerance rules.

The dequantizers restate the published GGML K-quant formats
(dequantize_row_q4_K / dequantize_row_q6_K of ggml-quants.c, the formats
the reference consumes: kernels/common.cu:40-84,164-186), vectorised over
blocks.  They share no code and no loop structure with oracle/oracle.c, so
agreement between the two pins the oracle's lane mapping, scale unpacking
and nibble/6-bit extraction.
"""
from __future__ import annotations

import numpy as np


# --------------------------------------------------------------- f16 helpers

def f16(bytes2: np.ndarray) -> np.ndarray:
    """uint8 [..., 2] little-endian -> float64."""
    return np.ascontiguousarray(bytes2).view(np.float16)[..., 0].astype(np.float64)


# --------------------------------------------------------------- Q4_K

def q4k_scales_mins(sc12: np.ndarray):
    """uint8 [n, 12] -> (sc [n, 8], m [n, 8]) per the GGML 6-bit packing."""
    s = sc12.astype(np.int64)
    sc = np.zeros((s.shape[0], 8), np.int64)
    m = np.zeros((s.shape[0], 8), np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def q4k_quants(blk: np.ndarray) -> np.ndarray:
    """uint8 [n, 144] -> 4-bit quants [n, 256] in value order."""
    qs = blk[:, 16:144].astype(np.int64).reshape(-1, 4, 32)  # [n, chunk, l]
    lo = qs & 0xF
    hi = qs >> 4
    return np.concatenate([lo, hi], axis=2).reshape(-1, 256)  # chunk j: lo then hi


def q4k_dequant(blk: np.ndarray) -> np.ndarray:
    """uint8 [n, 144] -> float64 [n, 256]."""
    d = f16(blk[:, 0:2].reshape(-1, 1, 2)).reshape(-1, 1)
    dmin = f16(blk[:, 2:4].reshape(-1, 1, 2)).reshape(-1, 1)
    sc, m = q4k_scales_mins(blk[:, 4:16])
    q = q4k_quants(blk)
    g = np.arange(256) // 32
    return d * sc[:, g] * q - dmin * m[:, g]


# --------------------------------------------------------------- Q6_K

def q6k_quants(blk: np.ndarray) -> np.ndarray:
    """uint8 [n, >=210] -> signed quants (q - 32) [n, 256] in value order."""
    ql = blk[:, 0:128].astype(np.int64).reshape(-1, 2, 64)
    qh = blk[:, 128:192].astype(np.int64).reshape(-1, 2, 32)
    out = np.zeros((blk.shape[0], 2, 4, 32), np.int64)
    out[:, :, 0] = (ql[:, :, 0:32] & 0xF) | (((qh >> 0) & 3) << 4)
    out[:, :, 1] = (ql[:, :, 32:64] & 0xF) | (((qh >> 2) & 3) << 4)
    out[:, :, 2] = (ql[:, :, 0:32] >> 4) | (((qh >> 4) & 3) << 4)
    out[:, :, 3] = (ql[:, :, 32:64] >> 4) | (((qh >> 6) & 3) << 4)
    return out.reshape(-1, 256) - 32


def q6k_dequant(blk: np.ndarray) -> np.ndarray:
    d = f16(blk[:, 208:210].reshape(-1, 1, 2)).reshape(-1, 1)
    sc = blk[:, 192:208].view(np.int8).astype(np.int64)
    return d * sc[:, np.arange(256) // 16] * q6k_quants(blk)


# --------------------------------------------------------------- Q8_0 / Q5_0

def q8_0_dequant(blk: np.ndarray) -> np.ndarray:
    """uint8 [n, 34] -> float64 [n, 32] (dequantize_row_q8_0: d * qs[t])."""
    d = f16(blk[:, 0:2].reshape(-1, 1, 2)).reshape(-1, 1)
    return d * np.ascontiguousarray(blk[:, 2:34]).view(np.int8).astype(np.float64)


def q5_0_dequant(blk: np.ndarray) -> np.ndarray:
    """uint8 [n, 22] -> float64 [n, 32] (dequantize_row_q5_0: value t < 16
    from the low nibble of qs[t], 16 + t from its high nibble; bit 4 of value
    v is bit v of the little-endian u32 qh; value = d * (code - 16))."""
    d = f16(blk[:, 0:2].reshape(-1, 1, 2)).reshape(-1, 1)
    qh = np.ascontiguousarray(blk[:, 2:6]).view("<u4").astype(np.int64)  # [n, 1]
    qs = blk[:, 6:22].astype(np.int64)
    nib = np.concatenate([qs & 15, qs >> 4], axis=1)
    hi = (qh >> np.arange(32)) & 1
    return d * (nib + 16 * hi - 16)


def gemv_block32_ref(w, n_rows, xvec, block_bytes):
    """fp64 W x for a 32-value block format (34: Q8_0, 22: Q5_0)."""
    nb = n_rows // 32
    blocks = w[:, : nb * block_bytes].reshape(-1, block_bytes)
    deq = q8_0_dequant if block_bytes == 34 else q5_0_dequant
    W = deq(blocks).reshape(w.shape[0], nb * 32)
    return W @ np.asarray(xvec, np.float64)[: nb * 32]


# --------------------------------------------------------------- matrices

def matrix_blocks(w: np.ndarray, n_rows: int, block_bytes: int) -> np.ndarray:
    """[n_cols, col_bytes] -> [n_cols, floor(n_rows/256), block_bytes]."""
    nb = n_rows // 256
    return w[:, : nb * block_bytes].reshape(w.shape[0], nb, block_bytes)


def q8_dequant(q8: np.ndarray, d8: np.ndarray) -> np.ndarray:
    return q8.astype(np.float64) * np.repeat(d8.astype(np.float64), 32)


def gemv_q4k_ref(w, n_rows, xvec):
    """fp64 y = W x with W dequantized per GGML (x: float64 of length >= nb*256)."""
    blocks = matrix_blocks(w, n_rows, 144)
    n_cols, nb = blocks.shape[:2]
    W = q4k_dequant(blocks.reshape(-1, 144)).reshape(n_cols, nb * 256)
    return W @ xvec[: nb * 256]


def gemv_q6k_ref(w, n_rows, xvec, block_bytes=210):
    blocks = matrix_blocks(w, n_rows, block_bytes)
    n_cols, nb = blocks.shape[:2]
    W = q6k_dequant(blocks.reshape(-1, block_bytes)).reshape(n_cols, nb * 256)
    return W @ xvec[: nb * 256]


def gemm_ref(fmt, w, n_rows, x):
    """fp64 (Y, sum |terms|) of the prefill GEMM Y[t] = W x[t] for a Q4_K
    ("q4k", 144-byte) or raw Q6_K ("q6k", 210-byte) matrix."""
    bb = 144 if fmt == "q4k" else 210
    blocks = matrix_blocks(w, n_rows, bb)
    n_cols, nb = blocks.shape[:2]
    deq = q4k_dequant if fmt == "q4k" else q6k_dequant
    W = deq(blocks.reshape(-1, bb)).reshape(n_cols, nb * 256)
    X = np.asarray(x, np.float64)[:, : nb * 256]
    return X @ W.T, np.abs(X) @ np.abs(W).T


# --------------------------------------------------------------- tolerances

GEMV_RTOL = 1e-5        # north-star fp32 GEMV tolerance (relative)
CANCEL_FLOOR = 0.1      # floor on |y| as a fraction of sum |terms|
ATTN_ATOL = 2e-3        # north-star attention tolerance (absolute)


def gemv_tol(y_ref: np.ndarray, rowabs: np.ndarray) -> np.ndarray:
    """Per-output tolerance: 1e-5 relative to max(|y|, 0.1 * sum|terms|).

    The floor keeps rows whose terms cancel (|y| much smaller than the terms
    it sums) from demanding more than fp32 can give; sum|terms| is the
    fp64 sum of the magnitudes of the per-sub-block scale and min terms.
    """
    return GEMV_RTOL * np.maximum(np.abs(y_ref), CANCEL_FLOOR * rowabs)


def assert_gemv_close(y, y_ref, rowabs, what=""):
    y = np.asarray(y, np.float64)
    tol = gemv_tol(y_ref, rowabs)
    err = np.abs(y - y_ref)
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, (
        f"{what}: {bad.size} outputs out of tolerance; worst j={bad[np.argmax(err[bad] / tol[bad])]}"
        f" err={err[bad].max():.3e} tol={tol[bad].min():.3e}")


def silu64(g):
    return g * np.exp(-np.logaddexp(0.0, -g))  # g / (1 + e^-g) without overflow


def assert_ffn_close(h, g64, ga, u64, ua, what="ffn"):
    """h = silu(g) * u with g, u carrying the GEMV tolerance; first-order
    propagation of 1e-5 relative errors in g, u, plus 1e-5 relative for the
    SiLU evaluation itself."""
    sig = np.exp(-np.logaddexp(0.0, -g64))  # 1 / (1 + e^-g) without overflow
    dsilu = sig * (1.0 + g64 * (1.0 - sig))
    ref = silu64(g64) * u64
    sg = np.maximum(np.abs(g64), CANCEL_FLOOR * ga)
    su = np.maximum(np.abs(u64), CANCEL_FLOOR * ua)
    tol = GEMV_RTOL * (np.abs(dsilu * u64) * sg + np.abs(silu64(g64)) * su + np.abs(ref))
    # exp(-g) overflows fp32 for g < -log(FLT_MAX): fp32 SiLU is then exactly
    # 0 (the reference's __expf overflows the same way) while fp64 is ~e^g.
    overflow = -g64 > np.log(np.finfo(np.float32).max)
    tol = np.where(overflow, np.maximum(tol, np.abs(ref) * (1 + GEMV_RTOL)), tol)
    err = np.abs(np.asarray(h, np.float64) - ref)
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, f"{what}: {bad.size} bad, worst err {err.max():.3e}"
