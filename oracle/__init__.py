"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

ctypes binding of oracle/liboracle.so, a plain-C restatement of the
reference kernels (see oracle.h for the per-function citations).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker or the CPU baseline; the product
library never calls it.

Parity pins (what fixes each function independently of this restatement) are
listed in the module docstrings of tests/test_oracle_*.py.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _lib.or_f16_to_f32.restype = C.c_float
        _lib.or_f16_to_f32.argtypes = [C.c_uint16]
        _lib.or_f32_to_f16_halfup.restype = C.c_uint16
        _lib.or_f32_to_f16_halfup.argtypes = [C.c_float]
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _f32(n):
    return np.zeros(n, np.float32)


# ------------------------------------------------------------------ helpers

def f16_to_f32(h: int) -> float:
    return lib().or_f16_to_f32(h)


def f32_to_f16_halfup(f: float) -> int:
    return lib().or_f32_to_f16_halfup(f)


def quantize_q8(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    q8 = np.zeros(x.size, np.int8)
    d8 = _f32(x.size // 32)
    lib().or_quantize_q8(_p(x), _p(q8), _p(d8), C.c_int(x.size))
    return q8, d8


def q4k_block_dots(col: np.ndarray, q8: np.ndarray, nsb: int):
    dots = np.zeros(nsb * 8, np.int32)
    sums = np.zeros(nsb * 8, np.int32)
    lib().or_q4k_block_dots(_p(col), _p(q8), C.c_int(nsb), _p(dots), _p(sums))
    return dots, sums


def q6k_block_dots(col: np.ndarray, block_bytes: int, q8: np.ndarray, nsb: int):
    dots = np.zeros(nsb * 16, np.int32)
    lib().or_q6k_block_dots(_p(col), C.c_int(block_bytes), _p(q8), C.c_int(nsb), _p(dots))
    return dots


def _res(use_res, residual, out):
    if use_res == 1:
        return np.ascontiguousarray(residual, np.float32)
    return None


# ------------------------------------------------------------------ GEMVs

def gemv_q4k_q8(w, xq, xd, n_rows, n_cols, col_bytes, bias=None, use_res=0,
                residual=None, out=None):
    out = _f32(n_cols) if out is None else np.array(out, np.float32)
    lib().or_gemv_q4k_q8(_p(w), _p(xq), _p(xd), _p(out), n_rows, n_cols, col_bytes,
                         int(bias is not None), _p(bias), use_res,
                         _p(_res(use_res, residual, out)))
    return out


def gemv_q4k_q8_splitk(w, xq, xd, n_rows, n_cols, col_bytes, n_split):
    part = _f32(n_split * n_cols)
    lib().or_gemv_q4k_q8_splitk(_p(w), _p(xq), _p(xd), _p(part), n_rows, n_cols,
                                col_bytes, n_split)
    return part


def gemv_splitk_reduce(partial, n_cols, n_split, bias=None, use_res=0, residual=None,
                       out=None):
    out = _f32(n_cols) if out is None else np.array(out, np.float32)
    lib().or_gemv_splitk_reduce(_p(partial), _p(out), n_cols, n_split,
                                int(bias is not None), _p(bias), use_res,
                                _p(_res(use_res, residual, out)))
    return out


def gemv_q4k_pair(wa, wb, xq, xd, n_rows, n_a, n_b, col_bytes, ba=None, bb=None):
    oa, ob = _f32(n_a), _f32(n_b)
    lib().or_gemv_q4k_pair(_p(wa), _p(wb), _p(xq), _p(xd), _p(oa), _p(ob), n_rows, n_a,
                           n_b, col_bytes, int(ba is not None), _p(ba), _p(bb))
    return oa, ob


def gemv_q4k_dual(wa, wb, xq, xd, n_rows, n_cols, col_bytes):
    oa, ob = _f32(n_cols), _f32(n_cols)
    lib().or_gemv_q4k_dual(_p(wa), _p(wb), _p(xq), _p(xd), _p(oa), _p(ob), n_rows, n_cols,
                           col_bytes)
    return oa, ob


def gemv_q4k_ffn(gate, up, xq, xd, n_rows, n_cols, col_bytes, ways=1):
    out = _f32(n_cols)
    lib().or_gemv_q4k_ffn(_p(gate), _p(up), _p(xq), _p(xd), _p(out), n_rows, n_cols,
                          col_bytes, ways)
    return out


def gemv_q4k_qkv(wq, wk, wv, xq, xd, n_rows, n_q, n_k, n_v, col_bytes, bq=None, bk=None,
                 bv=None):
    q, k, v = _f32(n_q), _f32(n_k), _f32(n_v)
    lib().or_gemv_q4k_qkv(_p(wq), _p(wk), _p(wv), _p(xq), _p(xd), _p(q), _p(k), _p(v),
                          n_rows, n_q, n_k, n_v, col_bytes, int(bq is not None), _p(bq),
                          _p(bk), _p(bv))
    return q, k, v


def gemv_q6k_compact_q8(w, xq, xd, n_rows, n_cols, col_bytes, bias=None, use_res=0,
                        residual=None, out=None):
    out = _f32(n_cols) if out is None else np.array(out, np.float32)
    lib().or_gemv_q6k_compact_q8(_p(w), _p(xq), _p(xd), _p(out), n_rows, n_cols, col_bytes,
                                 int(bias is not None), _p(bias), use_res,
                                 _p(_res(use_res, residual, out)))
    return out


def gemv_q6k_compact_q8_kway(w, xq, xd, n_rows, n_cols, col_bytes, ways=8, bias=None,
                             use_res=0, residual=None, out=None):
    out = _f32(n_cols) if out is None else np.array(out, np.float32)
    lib().or_gemv_q6k_compact_q8_kway(_p(w), _p(xq), _p(xd), _p(out), n_rows, n_cols,
                                      col_bytes, ways, int(bias is not None), _p(bias),
                                      use_res, _p(_res(use_res, residual, out)))
    return out


def gemv_q6k_compact_q8_splitk(w, xq, xd, n_rows, n_cols, col_bytes, n_split):
    part = _f32(n_split * n_cols)
    lib().or_gemv_q6k_compact_q8_splitk(_p(w), _p(xq), _p(xd), _p(part), n_rows, n_cols,
                                        col_bytes, n_split)
    return part


def gemv_q6k_f32(w, x, n_rows, n_cols, col_bytes, bias=None, use_res=0, residual=None,
                 out=None):
    out = _f32(n_cols) if out is None else np.array(out, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemv_q6k_f32(_p(w), _p(x), _p(out), n_rows, n_cols, col_bytes,
                          int(bias is not None), _p(bias), use_res,
                          _p(_res(use_res, residual, out)))
    return out


def q6k_compact_repack(raw, n_rows, n_cols, col_bytes):
    nb = n_rows // 256
    out = np.zeros(n_cols * nb * 212, np.uint8)
    lib().or_q6k_compact_repack(_p(raw), _p(out), n_rows, n_cols, col_bytes)
    return out.reshape(n_cols, nb * 212)


# ------------------------------------------------------------------ fp64 truth

def gemv_q4k_q8_f64(w, xq, xd, n_rows, n_cols, col_bytes):
    out = np.zeros(n_cols, np.float64)
    absn = np.zeros(n_cols, np.float64)
    lib().or_gemv_q4k_q8_f64(_p(w), _p(xq), _p(xd), _p(out), _p(absn), n_rows, n_cols,
                             col_bytes)
    return out, absn


def gemv_q6k_q8_f64(w, block_bytes, xq, xd, n_rows, n_cols, col_bytes):
    out = np.zeros(n_cols, np.float64)
    absn = np.zeros(n_cols, np.float64)
    lib().or_gemv_q6k_q8_f64(_p(w), block_bytes, _p(xq), _p(xd), _p(out), _p(absn), n_rows,
                             n_cols, col_bytes)
    return out, absn


def gemv_q6k_f32_f64(w, x, n_rows, n_cols, col_bytes):
    out = np.zeros(n_cols, np.float64)
    absn = np.zeros(n_cols, np.float64)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemv_q6k_f32_f64(_p(w), _p(x), _p(out), _p(absn), n_rows, n_cols, col_bytes)
    return out, absn


# ------------------------------------------------------ Q8_0 / Q5_0 GEMVs

def gemv_q8_0_q8(w, xq, xd, n_rows, n_cols, col_bytes, bias=None, use_res=0,
                 residual=None, out=None):
    out = _f32(n_cols) if out is None else np.array(out, np.float32)
    lib().or_gemv_q8_0_q8(_p(w), _p(xq), _p(xd), _p(out), n_rows, n_cols, col_bytes,
                          int(bias is not None), _p(bias), use_res,
                          _p(_res(use_res, residual, out)))
    return out


def gemv_q8_0_q8_splitk(w, xq, xd, n_rows, n_cols, col_bytes, n_split):
    part = _f32(n_split * n_cols)
    lib().or_gemv_q8_0_q8_splitk(_p(w), _p(xq), _p(xd), _p(part), n_rows, n_cols,
                                 col_bytes, n_split)
    return part


def gemv_q8_0_f32_splitk(w, x, n_rows, n_cols, col_bytes, n_split):
    part = _f32(n_split * n_cols)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemv_q8_0_f32_splitk(_p(w), _p(x), _p(part), n_rows, n_cols, col_bytes,
                                  n_split)
    return part


def gemv_q5_0_f32(w, x, n_rows, n_cols, col_bytes, bias=None, use_res=0, residual=None,
                  out=None):
    out = _f32(n_cols) if out is None else np.array(out, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemv_q5_0_f32(_p(w), _p(x), _p(out), n_rows, n_cols, col_bytes,
                           int(bias is not None), _p(bias), use_res,
                           _p(_res(use_res, residual, out)))
    return out


def gemv_q5_0_f32_splitk(w, x, n_rows, n_cols, col_bytes, n_split):
    part = _f32(n_split * n_cols)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemv_q5_0_f32_splitk(_p(w), _p(x), _p(part), n_rows, n_cols, col_bytes,
                                  n_split)
    return part


def q8_0_block_sums(w, xq, n_rows, n_cols, col_bytes):
    sums = np.zeros(n_cols * (n_rows // 32), np.int32)
    lib().or_q8_0_block_sums(_p(w), _p(xq), _p(sums), n_rows, n_cols, col_bytes)
    return sums.reshape(n_cols, -1)


def gemv_q8_0_q8_f64(w, xq, xd, n_rows, n_cols, col_bytes):
    out, absn = np.zeros(n_cols, np.float64), np.zeros(n_cols, np.float64)
    lib().or_gemv_q8_0_q8_f64(_p(w), _p(xq), _p(xd), _p(out), _p(absn), n_rows, n_cols,
                              col_bytes)
    return out, absn


def gemv_q8_0_f32_f64(w, x, n_rows, n_cols, col_bytes):
    out, absn = np.zeros(n_cols, np.float64), np.zeros(n_cols, np.float64)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemv_q8_0_f32_f64(_p(w), _p(x), _p(out), _p(absn), n_rows, n_cols, col_bytes)
    return out, absn


def gemv_q5_0_f32_f64(w, x, n_rows, n_cols, col_bytes):
    out, absn = np.zeros(n_cols, np.float64), np.zeros(n_cols, np.float64)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemv_q5_0_f32_f64(_p(w), _p(x), _p(out), _p(absn), n_rows, n_cols, col_bytes)
    return out, absn


# ------------------------------------------------------------- prefill GEMMs

def gemm_q4k(w, x, n_rows, n_cols, col_bytes, n_tok):
    out = _f32(n_tok * n_cols)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemm_q4k(_p(w), _p(x), _p(out), n_rows, n_cols, col_bytes, n_tok)
    return out.reshape(n_tok, n_cols)


def gemm_q6k(w, x, n_rows, n_cols, col_bytes, n_tok):
    out = _f32(n_tok * n_cols)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_gemm_q6k(_p(w), _p(x), _p(out), n_rows, n_cols, col_bytes, n_tok)
    return out.reshape(n_tok, n_cols)


# ------------------------------------------------------------------ attention

def attn_prefill(q, k_cache, v_cache, n_head, n_kv, head_dim, pos0, n_q, scale):
    out = _f32(n_q * n_head * head_dim)
    lib().or_attn_prefill(_p(np.ascontiguousarray(q, np.float32)), _p(k_cache), _p(v_cache),
                          _p(out), n_head, n_kv, head_dim, pos0, n_q, C.c_float(scale))
    return out.reshape(n_q, n_head * head_dim)


def flash_partial(q, k_cache, v_cache, n_head, n_kv, head_dim, pos0, n_split, scale):
    part = _f32(n_head * n_split * (2 + head_dim))
    q = np.ascontiguousarray(q, np.float32)
    lib().or_flash_partial(_p(q), _p(k_cache), _p(v_cache), _p(part), n_head, n_kv,
                           head_dim, pos0, n_split, C.c_float(scale))
    return part


def flash_reduce(partial, n_head, head_dim, n_split):
    out = _f32(n_head * head_dim)
    lib().or_flash_reduce(_p(partial), _p(out), n_head, head_dim, n_split)
    return out


def attn_f64(q, k_cache, v_cache, n_head, n_kv, head_dim, seq_len, scale):
    out = np.zeros(n_head * head_dim, np.float64)
    q = np.ascontiguousarray(q, np.float32)
    lib().or_attn_f64(_p(q), _p(k_cache), _p(v_cache), _p(out), n_head, n_kv, head_dim,
                      seq_len, C.c_float(scale))
    return out


# ------------------------------------------------------------------ decode glue

def embed_row(table, block_bytes, token, n_rows, col_bytes):
    out = _f32(n_rows)
    lib().or_embed_row(_p(table), block_bytes, token, n_rows, col_bytes, _p(out))
    return out


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = _f32(x.size)
    lib().or_rms_norm(_p(x), _p(w), _p(out), x.size, C.c_float(eps))
    return out


def rope_neox(x, n_heads, head_dim, pos, theta):
    x = np.array(x, np.float32)
    lib().or_rope_neox(_p(x), n_heads, head_dim, pos, C.c_float(theta))
    return x


def f32_to_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size, np.uint16)
    lib().or_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def argmax(x):
    x = np.ascontiguousarray(x, np.float32)
    return lib().or_argmax(_p(x), x.size)


# ------------------------------------------------------------------ CPU baseline

def gemv_q4k_q8_mt(w, xq, xd, n_rows, n_cols, col_bytes, nthreads):
    out = _f32(n_cols)
    lib().or_gemv_q4k_q8_mt(_p(w), _p(xq), _p(xd), _p(out), n_rows, n_cols, col_bytes,
                            nthreads)
    return out


def gemv_q4k_ffn_mt(gate, up, xq, xd, n_rows, n_cols, col_bytes, nthreads):
    out = _f32(n_cols)
    lib().or_gemv_q4k_ffn_mt(_p(gate), _p(up), _p(xq), _p(xd), _p(out), n_rows, n_cols,
                             col_bytes, nthreads)
    return out


def gemv_q6k_compact_q8_kway_mt(w, xq, xd, n_rows, n_cols, col_bytes, ways, nthreads):
    out = _f32(n_cols)
    lib().or_gemv_q6k_compact_q8_kway_mt(_p(w), _p(xq), _p(xd), _p(out), n_rows, n_cols,
                                         col_bytes, ways, nthreads)
    return out


def flash_partial_mt(q, k_cache, v_cache, n_head, n_kv, head_dim, pos0, n_split, scale,
                     nthreads):
    part = _f32(n_head * n_split * (2 + head_dim))
    q = np.ascontiguousarray(q, np.float32)
    lib().or_flash_partial_mt(_p(q), _p(k_cache), _p(v_cache), _p(part), n_head, n_kv,
                              head_dim, pos0, n_split, C.c_float(scale), nthreads)
    return part
