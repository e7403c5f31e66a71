"""Python handle on the C++ decode runtime (tf_model_* in include/taraference_hip.h).

Weights are uploaded to device tensors owned by this object; Q6_K matrices
that the Q8 path reads (ffn_down, lm_head) also get their 212-byte compact
copy, made on the device by tf_q6k_compact_repack (cuda/load.rs:145-159).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import capi, synth

TYPE_Q4_K = 12
TYPE_Q6_K = 14


class TfMat(C.Structure):
    _fields_ = [("data", C.c_void_p), ("compact", C.c_void_p), ("type", C.c_int),
                ("n_rows", C.c_int), ("n_cols", C.c_int), ("col_bytes", C.c_int),
                ("compact_col_bytes", C.c_int)]


class TfLayer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("wq", TfMat), ("wk", TfMat), ("wv", TfMat),
                ("bq", C.c_void_p), ("bk", C.c_void_p), ("bv", C.c_void_p), ("wo", TfMat),
                ("ffn_norm", C.c_void_p), ("gate", TfMat), ("up", TfMat), ("down", TfMat)]


class TfModelConfig(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("n_embd", C.c_int), ("n_ff", C.c_int),
                ("n_head", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
                ("n_vocab", C.c_int), ("max_seq", C.c_int), ("rope_theta", C.c_float),
                ("rms_eps", C.c_float)]


def _bind(lib):
    lib.tf_model_create.argtypes = [C.POINTER(TfModelConfig), C.POINTER(TfLayer),
                                    C.POINTER(TfMat), C.POINTER(TfMat), C.c_void_p,
                                    C.POINTER(C.c_void_p)]
    lib.tf_model_create.restype = C.c_int
    lib.tf_model_destroy.argtypes = [C.c_void_p]
    lib.tf_model_destroy.restype = None
    lib.tf_model_forward.argtypes = [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_int),
                                     C.c_void_p]
    lib.tf_model_forward.restype = C.c_int
    lib.tf_model_generate.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.c_int, C.c_int,
                                      C.c_int, C.POINTER(C.c_int), C.c_int, C.c_void_p]
    lib.tf_model_generate.restype = C.c_int
    lib.tf_model_set_path.argtypes = [C.c_void_p, C.c_int]
    lib.tf_model_set_path.restype = C.c_int
    lib.tf_model_get_path.argtypes = [C.c_void_p]
    lib.tf_model_get_path.restype = C.c_int
    lib.tf_model_logits.argtypes = [C.c_void_p]
    lib.tf_model_logits.restype = C.c_void_p
    for n in ("tf_model_k_cache", "tf_model_v_cache"):
        getattr(lib, n).argtypes = [C.c_void_p, C.c_int]
        getattr(lib, n).restype = C.c_void_p


class DecodeModel:
    """Greedy batch-1 decoder over caller-supplied synthetic weights.

    cfg: dict with n_layer, n_embd, n_ff, n_head, n_kv, head_dim, n_vocab,
    rope_theta, rms_eps and max_seq.  layers: iterable of synth.qwen_layer()
    dicts (consumed one at a time, so host memory holds one layer).
    embedding: (raw Q6_K bytes [n_vocab, col_bytes], col_bytes), tied lm_head.
    """

    def __init__(self, cfg: dict, layers, embedding):
        self.lib = capi.load()
        _bind(self.lib)
        self.cfg = dict(cfg)
        self._keep = []
        self.stream = capi.stream_ptr()
        c = self.cfg
        carr = (TfLayer * c["n_layer"])()
        for li, L in enumerate(layers):
            t = carr[li]
            t.attn_norm = self._f32(L["attn_norm"])
            t.ffn_norm = self._f32(L["ffn_norm"])
            t.wq = self._q4(L["wq"], c["n_embd"])
            t.wk = self._q4(L["wk"], c["n_embd"])
            t.wv = self._q6(L["wv"], c["n_embd"], compact=False)
            t.bq, t.bk, t.bv = self._f32(L["bq"]), self._f32(L["bk"]), self._f32(L["bv"])
            t.wo = self._q4(L["wo"], c["n_head"] * c["head_dim"])
            t.gate = self._q4(L["gate"], c["n_embd"])
            t.up = self._q4(L["up"], c["n_embd"])
            t.down = (self._q6(L["down"], c["n_ff"], compact=True) if L["down_q6k"]
                      else self._q4(L["down"], c["n_ff"]))
        self.embd = self._q6(embedding, c["n_embd"], compact=True)
        self.output_norm = self._f32(np.ones(c["n_embd"], np.float32))
        cc = TfModelConfig(c["n_layer"], c["n_embd"], c["n_ff"], c["n_head"], c["n_kv"],
                           c["head_dim"], c["n_vocab"], c["max_seq"], c["rope_theta"],
                           c["rms_eps"])
        h = C.c_void_p()
        rc = self.lib.tf_model_create(C.byref(cc), carr, C.byref(self.embd), C.byref(self.embd),
                                      self.output_norm, C.byref(h))
        if rc != 0:
            raise capi.HipError(f"tf_model_create returned {rc}")
        self.h = h
        self._layers = carr

    # ---------------------------------------------------------------- upload
    def _dev(self, a: np.ndarray) -> torch.Tensor:
        t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
        self._keep.append(t)
        return t

    def _f32(self, a) -> int:
        return self._dev(np.asarray(a, np.float32)).data_ptr()

    def _q4(self, wm, n_rows) -> TfMat:
        w, cb = wm
        return TfMat(self._dev(w).data_ptr(), None, TYPE_Q4_K, n_rows, w.shape[0], cb, 0)

    def _q6(self, wm, n_rows, compact: bool) -> TfMat:
        w, cb = wm
        raw = self._dev(w)
        comp, ccb = None, 0
        if compact:
            nb = n_rows // 256
            ccb = nb * synth.Q6K_COMPACT_BYTES
            comp = torch.empty(w.shape[0] * ccb, dtype=torch.uint8, device="cuda")
            self._keep.append(comp)
            capi.call("tf_q6k_compact_repack", raw.data_ptr(), comp.data_ptr(), n_rows,
                      w.shape[0], cb, self.stream)
        return TfMat(raw.data_ptr(), comp.data_ptr() if comp is not None else None, TYPE_Q6_K,
                     n_rows, w.shape[0], cb, ccb)

    # ---------------------------------------------------------------- decode
    def forward(self, token: int, pos: int) -> int:
        """One eager decode step at position pos; returns the argmax token."""
        nxt = C.c_int()
        rc = self.lib.tf_model_forward(self.h, token, pos, C.byref(nxt), self.stream)
        if rc != 0:
            raise capi.HipError(f"tf_model_forward returned {rc}")
        return nxt.value

    def set_path(self, path: int) -> None:
        """0 = reference kernel sequence, 1 = fused (quantize once),
        2 = fused with GEMV prologues, 3 = as 2 with a separate h quantize
        (default), 4 = the whole step in one persistent launch."""
        rc = self.lib.tf_model_set_path(self.h, int(path))
        if rc != 0:
            raise capi.HipError(f"tf_model_set_path returned {rc}")

    def path(self) -> int:
        """The decode path in use (4 = persistent step, the default where it
        applies)."""
        return int(self.lib.tf_model_get_path(self.h))

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg["n_vocab"], np.float32)
        torch.cuda.synchronize()
        capi.memcpy_d2h(out, self.lib.tf_model_logits(self.h))
        return out

    def kv_cache(self, layer: int, seq: int):
        """(K, V) f16 bits [seq, n_kv*head_dim] of one layer, copied to the host."""
        n = seq * self.cfg["n_kv"] * self.cfg["head_dim"]
        k, v = np.empty(n, np.uint16), np.empty(n, np.uint16)
        torch.cuda.synchronize()
        capi.memcpy_d2h(k, self.lib.tf_model_k_cache(self.h, layer))
        capi.memcpy_d2h(v, self.lib.tf_model_v_cache(self.h, layer))
        return k.reshape(seq, -1), v.reshape(seq, -1)

    def generate(self, forced, n_gen: int, pos0: int = 0, use_graph: bool = True):
        """Feed `forced` through the decode path, then n_gen greedy steps;
        returns the greedy continuation (n_gen tokens)."""
        forced = np.ascontiguousarray(forced, np.int32)
        arr = (C.c_int * len(forced))(*forced.tolist())
        out = (C.c_int * max(1, n_gen))()
        rc = self.lib.tf_model_generate(self.h, arr, len(forced), pos0, n_gen, out,
                                        int(use_graph), self.stream)
        if rc != 0:
            raise capi.HipError(f"tf_model_generate returned {rc}")
        return np.array(out[:n_gen], np.int32)

    def close(self):
        if getattr(self, "h", None):
            torch.cuda.synchronize()
            self.lib.tf_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
