"""Seeded synthetic K-quant weights and activations.

Block formats follow the GGUF / reference layout (kernels/common.cu:40-186):
  Q4_K, 144 B: d f16, dmin f16, 12 packed 6-bit scale/min bytes, 128 qs bytes.
  Q6_K, 210 B: ql[128], qh[64], int8 scales[16], d f16.
  Q8_0, 34 B (32 values): d f16, int8 qs[32].
  Q5_0, 22 B (32 values): d f16, u32 qh, qs[16] (value t < 16 in the low
  nibble of qs[t], value 16 + t in its high nibble, bit 4 of value v in bit v
  of qh).
Distributions: d and dmin ~ U[1e-3, 1e-2] as f16;
6-bit scales and mins ~ U{0..63}; nibbles ~ U{0..15}; Q6_K ql/qh bytes
uniform, scales ~ U[-32, 31]; activations ~ N(0, 1) f32.

A weight matrix is returned as uint8 [n_cols, col_bytes]: output column j is
the contiguous run of ceil(n_rows/256) super-blocks, as the reference stores
it (cuda/load.rs:205-206,235).
"""
from __future__ import annotations

import numpy as np

Q4K_BYTES = 144
Q6K_BYTES = 210
Q6K_COMPACT_BYTES = 212
Q8_0_BYTES = 34
Q5_0_BYTES = 22

SEED_BASE = 0x7A7A0000


def rng_for(config: int, salt: int = 0) -> np.random.Generator:
    return np.random.default_rng(SEED_BASE + config * 1000 + salt)


def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Pack 6-bit scales/mins [n, 8] into the 12-byte Q4_K layout.

    Inverse of get_scale_min_k4 (kernels/common.cu:40-50): for j < 4 the low
    six bits of bytes j and j+4 hold sc_j and m_j; for j >= 4 byte j+4 holds
    the low nibbles of sc_j | m_j << 4 and the top two bits of sc_j / m_j go
    to bits 6-7 of bytes j-4 / j.
    """
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.zeros((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = m[:, 0:4] | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    return out


def q4k_blocks(rng: np.random.Generator, n: int) -> np.ndarray:
    """n random Q4_K super-blocks as uint8 [n, 144]."""
    blk = np.empty((n, Q4K_BYTES), np.uint8)
    d = rng.uniform(1e-3, 1e-2, n).astype(np.float16)
    dmin = rng.uniform(1e-3, 1e-2, n).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(n, 2)
    sc = rng.integers(0, 64, (n, 8), dtype=np.uint8)
    m = rng.integers(0, 64, (n, 8), dtype=np.uint8)
    blk[:, 4:16] = pack_q4k_scales(sc, m)
    blk[:, 16:] = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    return blk


def q6k_blocks(rng: np.random.Generator, n: int) -> np.ndarray:
    """n random Q6_K super-blocks as uint8 [n, 210]."""
    blk = np.empty((n, Q6K_BYTES), np.uint8)
    blk[:, 0:192] = rng.integers(0, 256, (n, 192), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-32, 32, (n, 16), dtype=np.int8).view(np.uint8)
    d = rng.uniform(1e-3, 1e-2, n).astype(np.float16)
    blk[:, 208:210] = d.view(np.uint8).reshape(n, 2)
    return blk


def q4k_blocks_wc(rng: np.random.Generator, n: int) -> np.ndarray:
    """n well-conditioned Q4_K super-blocks: d ~ U[1e-4, 4e-4], sc ~ U{0..33},
    m = round(1.875 sc), dmin = 4 d, so each 32-value sub-block's mean
    d sc 7.5 - dmin m is about 0 and a weight's spread is about 0.02: a
    2048-wide GEMV of an RMS-1 input gives outputs of RMS about 1."""
    blk = np.empty((n, Q4K_BYTES), np.uint8)
    d = rng.uniform(1e-4, 4e-4, n).astype(np.float16)
    dmin = (d.astype(np.float32) * 4).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(n, 2)
    sc = rng.integers(0, 34, (n, 8), dtype=np.uint8)
    m = np.rint(sc * 1.875).astype(np.uint8)
    blk[:, 4:16] = pack_q4k_scales(sc, m)
    blk[:, 16:] = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    return blk


def q6k_blocks_wc(rng: np.random.Generator, n: int) -> np.ndarray:
    """n well-conditioned Q6_K super-blocks: scales ~ U[-8, 7], d ~ U[1e-4,
    4e-4] (weights of spread about 0.02)."""
    blk = np.empty((n, Q6K_BYTES), np.uint8)
    blk[:, 0:192] = rng.integers(0, 256, (n, 192), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-8, 8, (n, 16), dtype=np.int8).view(np.uint8)
    d = rng.uniform(1e-4, 4e-4, n).astype(np.float16)
    blk[:, 208:210] = d.view(np.uint8).reshape(n, 2)
    return blk


def q4k_matrix(rng, n_rows: int, n_cols: int, wc: bool = False) -> tuple[np.ndarray, int]:
    """Q4_K matrix [n_cols, col_bytes]; col_bytes = ceil(n_rows/256)*144
    (wc: the well-conditioned distribution of q4k_blocks_wc)."""
    nb = (n_rows + 255) // 256
    w = (q4k_blocks_wc if wc else q4k_blocks)(rng, n_cols * nb).reshape(n_cols, nb * Q4K_BYTES)
    return np.ascontiguousarray(w), nb * Q4K_BYTES


def q6k_matrix(rng, n_rows: int, n_cols: int, wc: bool = False) -> tuple[np.ndarray, int]:
    """Raw Q6_K matrix [n_cols, col_bytes]; col_bytes = ceil(n_rows/256)*210
    (wc: the well-conditioned distribution of q6k_blocks_wc)."""
    nb = (n_rows + 255) // 256
    w = (q6k_blocks_wc if wc else q6k_blocks)(rng, n_cols * nb).reshape(n_cols, nb * Q6K_BYTES)
    return np.ascontiguousarray(w), nb * Q6K_BYTES


def q6k_compact(raw: np.ndarray, n_rows: int) -> tuple[np.ndarray, int]:
    """Host restatement of cuda/load.rs:145-159 (210 -> 212-byte blocks)."""
    n_cols = raw.shape[0]
    nb = n_rows // 256
    out = np.zeros((n_cols, nb, Q6K_COMPACT_BYTES), np.uint8)
    out[:, :, :Q6K_BYTES] = raw[:, : nb * Q6K_BYTES].reshape(n_cols, nb, Q6K_BYTES)
    return out.reshape(n_cols, nb * Q6K_COMPACT_BYTES), nb * Q6K_COMPACT_BYTES


def q8_0_pack(d: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Q8_0 blocks [n, 34] from f16 scales d [n] and int8 values q [n, 32]."""
    n = q.shape[0]
    blk = np.empty((n, Q8_0_BYTES), np.uint8)
    blk[:, 0:2] = np.asarray(d, np.float16).view(np.uint8).reshape(n, 2)
    blk[:, 2:] = np.asarray(q, np.int8).view(np.uint8)
    return blk


def q5_0_pack(d: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Q5_0 blocks [n, 22] from f16 scales d [n] and 5-bit codes q [n, 32]
    (0..31; the value is d * (q - 16))."""
    q = np.asarray(q, np.uint32)
    n = q.shape[0]
    blk = np.empty((n, Q5_0_BYTES), np.uint8)
    blk[:, 0:2] = np.asarray(d, np.float16).view(np.uint8).reshape(n, 2)
    qh = ((q >> 4) << np.arange(32, dtype=np.uint32)).sum(axis=1, dtype=np.uint32)
    blk[:, 2:6] = qh.astype("<u4").view(np.uint8).reshape(n, 4)
    blk[:, 6:] = ((q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)).astype(np.uint8)
    return blk


def q8_0_matrix(rng, n_rows: int, n_cols: int) -> tuple[np.ndarray, int]:
    """Q8_0 matrix [n_cols, col_bytes]; col_bytes = n_rows/32 * 34; d ~ U[1e-3,
    1e-2] as f16, values ~ U{-127..127}."""
    nb = n_rows // 32
    d = rng.uniform(1e-3, 1e-2, n_cols * nb).astype(np.float16)
    q = rng.integers(-127, 128, (n_cols * nb, 32), dtype=np.int8)
    return np.ascontiguousarray(q8_0_pack(d, q).reshape(n_cols, nb * Q8_0_BYTES)), \
        nb * Q8_0_BYTES


def q5_0_matrix(rng, n_rows: int, n_cols: int) -> tuple[np.ndarray, int]:
    """Q5_0 matrix [n_cols, col_bytes]; col_bytes = n_rows/32 * 22; codes
    ~ U{0..31}."""
    nb = n_rows // 32
    d = rng.uniform(1e-3, 1e-2, n_cols * nb).astype(np.float16)
    q = rng.integers(0, 32, (n_cols * nb, 32), dtype=np.uint8)
    return np.ascontiguousarray(q5_0_pack(d, q).reshape(n_cols, nb * Q5_0_BYTES)), \
        nb * Q5_0_BYTES


def activation(rng, n: int) -> np.ndarray:
    return rng.standard_normal(n).astype(np.float32)


def kv_cache(rng, seq: int, n_kv: int, head_dim: int) -> np.ndarray:
    """f16 cache [seq, n_kv*head_dim] ~ N(0,1), returned as uint16 bits."""
    return rng.standard_normal((seq, n_kv * head_dim)).astype(np.float16).view(np.uint16)


# --------------------------------------------------------------- whole model

QWEN25_3B = dict(n_layer=36, n_embd=2048, n_ff=11008, n_head=16, n_kv=2, head_dim=128,
                 n_vocab=151936, rope_theta=1e6, rms_eps=1e-6)
QWEN25_7B = dict(n_layer=28, n_embd=3584, n_ff=18944, n_head=28, n_kv=4, head_dim=128,
                 n_vocab=152064, rope_theta=1e6, rms_eps=1e-6)


def down_is_q6k(layer: int) -> bool:
    """Q4_K_M placement used for the synthetic models: ffn_down is Q6_K on
    odd layers (alternate layers), Q4_K on even ones."""
    return layer % 2 == 1


def qwen_layer(rng, cfg: dict, layer: int, wc: bool = False) -> dict:
    """Random-init weights of one dense Qwen2 layer in the Q4_K_M mix:
    Q4_K for q/k/o/gate/up, Q6_K for v, Q6_K or Q4_K for down; norms = 1,
    q/k/v biases ~ N(0, 0.02).  wc: well-conditioned blocks (activations,
    attention scores and logits of order 1, so the softmax is not one-hot)
    instead of the plain random block distribution (the bench draws wc)."""
    e, f = cfg["n_embd"], cfg["n_ff"]
    nq = cfg["n_head"] * cfg["head_dim"]
    nkv = cfg["n_kv"] * cfg["head_dim"]
    L = {}
    L["attn_norm"] = np.ones(e, np.float32)
    L["ffn_norm"] = np.ones(e, np.float32)
    L["wq"] = q4k_matrix(rng, e, nq, wc)
    L["wk"] = q4k_matrix(rng, e, nkv, wc)
    L["wv"] = q6k_matrix(rng, e, nkv, wc)
    L["bq"] = (rng.standard_normal(nq) * 0.02).astype(np.float32)
    L["bk"] = (rng.standard_normal(nkv) * 0.02).astype(np.float32)
    L["bv"] = (rng.standard_normal(nkv) * 0.02).astype(np.float32)
    L["wo"] = q4k_matrix(rng, nq, e, wc)
    L["gate"] = q4k_matrix(rng, e, f, wc)
    L["up"] = q4k_matrix(rng, e, f, wc)
    L["down"] = q6k_matrix(rng, f, e, wc) if down_is_q6k(layer) else q4k_matrix(rng, f, e, wc)
    L["down_q6k"] = down_is_q6k(layer)
    return L


def qwen_embedding(rng, cfg: dict, wc: bool = False):
    """Tied token embedding / lm_head: Q6_K [n_vocab, n_embd]."""
    return q6k_matrix(rng, cfg["n_embd"], cfg["n_vocab"], wc)


def weight_bytes(cfg: dict) -> int:
    """GGUF bytes streamed per decode token (lm_head counted once, embedding
    row not counted)."""
    e, f, hd = cfg["n_embd"], cfg["n_ff"], cfg["head_dim"]
    nq, nkv = cfg["n_head"] * hd, cfg["n_kv"] * hd
    q4 = lambda k, n: n * (k // 256) * Q4K_BYTES  # noqa: E731
    q6 = lambda k, n: n * (k // 256) * Q6K_BYTES  # noqa: E731
    tot = 0
    for li in range(cfg["n_layer"]):
        tot += q4(e, nq) + q4(e, nkv) + q6(e, nkv) + q4(nq, e) + 2 * q4(e, f)
        tot += q6(f, e) if down_is_q6k(li) else q4(f, e)
    tot += q6(e, cfg["n_vocab"])
    return tot


QWEN25_05B = dict(n_layer=24, n_embd=896, n_ff=4864, n_head=14, n_kv=2, head_dim=64,
                  n_vocab=151936, rope_theta=1e6, rms_eps=1e-6)


def qwen05_layer(rng, cfg: dict, layer: int) -> dict:
    """Random-init weights of one Qwen2.5-0.5B-layout layer as a Q4_K_M file
    stores them when the hidden width (896) is not a multiple of 256: the
    896-row matrices fall back to Q5_0 (q/k/o/gate/up) and Q8_0 (v); down
    (4864 rows) stays Q4_K / Q6_K.  Matrices are (bytes, col_bytes, ggml type)."""
    e, f = cfg["n_embd"], cfg["n_ff"]
    nq = cfg["n_head"] * cfg["head_dim"]
    nkv = cfg["n_kv"] * cfg["head_dim"]

    def t(m, typ):
        return (m[0], m[1], typ)

    L = {}
    L["attn_norm"] = np.ones(e, np.float32)
    L["ffn_norm"] = np.ones(e, np.float32)
    L["wq"] = t(q5_0_matrix(rng, e, nq), 6)
    L["wk"] = t(q5_0_matrix(rng, e, nkv), 6)
    L["wv"] = t(q8_0_matrix(rng, e, nkv), 8)
    L["bq"] = (rng.standard_normal(nq) * 0.02).astype(np.float32)
    L["bk"] = (rng.standard_normal(nkv) * 0.02).astype(np.float32)
    L["bv"] = (rng.standard_normal(nkv) * 0.02).astype(np.float32)
    L["wo"] = t(q5_0_matrix(rng, nq, e), 6)
    L["gate"] = t(q5_0_matrix(rng, e, f), 6)
    L["up"] = t(q5_0_matrix(rng, e, f), 6)
    L["down_q6k"] = down_is_q6k(layer)
    L["down"] = t(q6k_matrix(rng, f, e), 14) if L["down_q6k"] else t(q4k_matrix(rng, f, e), 12)
    return L


def qwen05_embedding(rng, cfg: dict):
    """Tied token embedding / lm_head of the 0.5B layout: Q8_0 [n_vocab, n_embd]."""
    w, cb = q8_0_matrix(rng, cfg["n_embd"], cfg["n_vocab"])
    return (w, cb, 8)
