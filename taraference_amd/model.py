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
TYPE_Q5_0 = 6   # 32-value block formats: run on path 0 (the reference sequence)
TYPE_Q8_0 = 8


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
    lib.tf_model_prefill.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.c_int, C.c_int,
                                     C.POINTER(C.c_int), C.c_void_p]
    lib.tf_model_prefill.restype = C.c_int
    lib.tf_model_set_path.argtypes = [C.c_void_p, C.c_int]
    lib.tf_model_set_path.restype = C.c_int
    lib.tf_model_get_path.argtypes = [C.c_void_p]
    lib.tf_model_get_path.restype = C.c_int
    lib.tf_model_keep_stage_vectors.argtypes = [C.c_void_p, C.c_int]
    lib.tf_model_keep_stage_vectors.restype = C.c_int
    lib.tf_model_stage_vector.argtypes = [C.c_void_p, C.c_int, C.c_int]
    lib.tf_model_stage_vector.restype = C.c_void_p
    lib.tf_model_q8_record.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int]
    lib.tf_model_q8_record.restype = C.c_void_p
    lib.tf_model_logits.argtypes = [C.c_void_p]
    lib.tf_model_logits.restype = C.c_void_p
    for n in ("tf_model_k_cache", "tf_model_v_cache"):
        getattr(lib, n).argtypes = [C.c_void_p, C.c_int]
        getattr(lib, n).restype = C.c_void_p


class DecodeModel:
    """Greedy batch-1 decoder over caller-supplied weights.

    cfg: dict with n_layer, n_embd, n_ff, n_head, n_kv, head_dim, n_vocab,
    rope_theta, rms_eps and max_seq.  layers: iterable of per-layer dicts
    (synth.qwen_layer() or the GGUF loader; consumed one at a time, so host
    memory holds one layer).  A matrix is (bytes [n_cols, col_bytes],
    col_bytes) in the synthetic Q4_K_M placement (attn_v Q6_K, ffn_down Q6_K
    when down_q6k), or (bytes, col_bytes, ggml type).  Biases may be None.
    embedding: the token table (a matrix, Q6_K unless typed); output: a
    separate lm_head (None: tied to the embedding); output_norm: the final
    RMSNorm weight (None: ones).
    """

    @classmethod
    def from_gguf(cls, path, max_seq: int) -> "DecodeModel":
        """cuda/load.rs:166-420 for a dense Qwen2/Llama Q4_K_M file: the
        config from the metadata (config.rs:107-175), blk.{i}.* tensors by
        the reference's names, a tied lm_head when output.weight is absent."""
        from .gguf import GGML_F16, GGML_F32, GGML_Q4_K, GGML_Q6_K, GgufFile, ggml_nbytes

        f = GgufFile(path)
        try:
            cfg = f.model_config(max_seq)

            def mat(name, n_rows):
                t = f.tensor(name)
                if t is None:
                    raise ValueError(f"{path}: missing tensor {name}")
                if t.type not in (GGML_Q4_K, GGML_Q6_K, TYPE_Q5_0, TYPE_Q8_0):
                    raise ValueError(f"{name}: ggml type {t.type} is not on the decode path "
                                     "(Q4_K, Q6_K, Q5_0 and Q8_0 are)")
                if t.n_dims != 2 or t.dims[0] != n_rows:
                    raise ValueError(f"{name}: dims {list(t.dims[:t.n_dims])}, expected "
                                     f"[{n_rows}, n]")
                cb = ggml_nbytes(t.type, t.dims[0])
                return f.tensor_data(t).reshape(int(t.dims[1]), cb), cb, t.type

            def vec(name, n, required=True):
                t = f.tensor(name)
                if t is None:
                    if required:
                        raise ValueError(f"{path}: missing tensor {name}")
                    return None
                raw = f.tensor_data(t)
                if t.type == GGML_F32:
                    v = raw.view(np.float32)
                elif t.type == GGML_F16:
                    v = raw.view(np.float16).astype(np.float32)
                else:
                    raise ValueError(f"{name}: ggml type {t.type}, expected F32/F16")
                if v.size != n:
                    raise ValueError(f"{name}: {v.size} values, expected {n}")
                return v

            c = cfg
            qd, kvd = c["n_head"] * c["head_dim"], c["n_kv"] * c["head_dim"]

            def layers():
                for i in range(c["n_layer"]):
                    p = f"blk.{i}"
                    ffn_norm = vec(f"{p}.ffn_norm.weight", c["n_embd"], required=False)
                    if ffn_norm is None:
                        ffn_norm = vec(f"{p}.post_attention_norm.weight", c["n_embd"])
                    yield {
                        "attn_norm": vec(f"{p}.attn_norm.weight", c["n_embd"]),
                        "ffn_norm": ffn_norm,
                        "wq": mat(f"{p}.attn_q.weight", c["n_embd"]),
                        "wk": mat(f"{p}.attn_k.weight", c["n_embd"]),
                        "wv": mat(f"{p}.attn_v.weight", c["n_embd"]),
                        "bq": vec(f"{p}.attn_q.bias", qd, required=False),
                        "bk": vec(f"{p}.attn_k.bias", kvd, required=False),
                        "bv": vec(f"{p}.attn_v.bias", kvd, required=False),
                        "wo": mat(f"{p}.attn_output.weight", qd),
                        "gate": mat(f"{p}.ffn_gate.weight", c["n_embd"]),
                        "up": mat(f"{p}.ffn_up.weight", c["n_embd"]),
                        "down": mat(f"{p}.ffn_down.weight", c["n_ff"]),
                    }

            emb = mat("token_embd.weight", c["n_embd"])
            out = mat("output.weight", c["n_embd"]) if f.tensor("output.weight") else None
            return cls(cfg, layers(), emb, output=out,
                       output_norm=vec("output_norm.weight", c["n_embd"]))
        finally:
            f.close()

    def __init__(self, cfg: dict, layers, embedding, output=None, output_norm=None):
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
            t.wq = self._mat(L["wq"], c["n_embd"], TYPE_Q4_K)
            t.wk = self._mat(L["wk"], c["n_embd"], TYPE_Q4_K)
            t.wv = self._mat(L["wv"], c["n_embd"], TYPE_Q6_K, compact=False)
            t.bq, t.bk, t.bv = (self._f32(L.get(k)) for k in ("bq", "bk", "bv"))
            t.wo = self._mat(L["wo"], c["n_head"] * c["head_dim"], TYPE_Q4_K)
            t.gate = self._mat(L["gate"], c["n_embd"], TYPE_Q4_K)
            t.up = self._mat(L["up"], c["n_embd"], TYPE_Q4_K)
            t.down = self._mat(L["down"], c["n_ff"],
                               TYPE_Q6_K if L.get("down_q6k") else TYPE_Q4_K, compact=True)
        self.embd = self._mat(embedding, c["n_embd"], TYPE_Q6_K, compact=True)
        self.out = (self.embd if output is None
                    else self._mat(output, c["n_embd"], TYPE_Q6_K, compact=True))
        self.output_norm = self._f32(np.ones(c["n_embd"], np.float32) if output_norm is None
                                     else output_norm)
        cc = TfModelConfig(c["n_layer"], c["n_embd"], c["n_ff"], c["n_head"], c["n_kv"],
                           c["head_dim"], c["n_vocab"], c["max_seq"], c["rope_theta"],
                           c["rms_eps"])
        h = C.c_void_p()
        rc = self.lib.tf_model_create(C.byref(cc), carr, C.byref(self.embd), C.byref(self.out),
                                      self.output_norm, C.byref(h))
        if rc != 0:
            raise capi.HipError(f"tf_model_create returned {rc}")
        self.h = h
        self._layers = carr

    # ---------------------------------------------------------------- upload
    def _dev(self, a: np.ndarray) -> torch.Tensor:
        a = np.ascontiguousarray(a)
        if not a.flags.writeable:  # a view of a mapped file: copy (one matrix at a time)
            a = a.copy()
        t = torch.from_numpy(a).to("cuda")
        self._keep.append(t)
        return t

    def _f32(self, a) -> int | None:
        if a is None:
            return None
        return self._dev(np.asarray(a, np.float32)).data_ptr()

    def _mat(self, wm, n_rows, default_type, compact: bool = False) -> TfMat:
        """A matrix (bytes, col_bytes[, ggml type]); Q6_K ones the Q8 path reads
        (compact=True) also get the 212-byte repack."""
        typ = wm[2] if len(wm) > 2 else default_type
        w = (wm[0], wm[1])
        if typ == TYPE_Q4_K:
            return self._q4(w, n_rows)
        if typ == TYPE_Q6_K:
            return self._q6(w, n_rows, compact)
        if typ in (TYPE_Q5_0, TYPE_Q8_0):
            return TfMat(self._dev(w[0]).data_ptr(), None, typ, n_rows, w[0].shape[0], w[1], 0)
        raise ValueError(f"ggml type {typ} is not supported on the decode path")

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

    def keep_stage_vectors(self, on: bool = True) -> None:
        """Make the persistent step (path 4) keep every layer's stage vectors
        for stage_vector(); call before the first path-4 step."""
        rc = self.lib.tf_model_keep_stage_vectors(self.h, int(on))
        if rc != 0:
            raise capi.HipError(f"tf_model_keep_stage_vectors returned {rc}")

    STAGE_XA, STAGE_XB, STAGE_Q, STAGE_O, STAGE_H = 0, 1, 2, 4, 5
    Q8_QKV_IN, Q8_ATTN, Q8_GU_IN, Q8_H = 0, 1, 2, 3

    def q8_record(self, site: int, layer: int):
        """What the last persistent step's quantizer at `site` consumed and
        produced in layer `layer` (layer n_layer, site Q8_QKV_IN: the lm_head
        input): (f32 x[n], int8 q[n], f32 d[n/32]).  Needs keep_stage_vectors."""
        c = self.cfg
        n = {0: c["n_embd"], 1: c["n_head"] * c["head_dim"], 2: c["n_embd"], 3: c["n_ff"]}[site]
        ptrs = [self.lib.tf_model_q8_record(self.h, site, layer, part) for part in range(3)]
        if not all(ptrs):
            raise capi.HipError("no Q8 record (keep_stage_vectors before the step)")
        x = np.empty(n, np.float32)
        q = np.empty(n, np.int8)
        d = np.empty(n // 32, np.float32)
        torch.cuda.synchronize()
        for arr, p in zip((x, q, d), ptrs):
            capi.memcpy_d2h(arr, p)
        return x, q, d

    def stage_vector(self, kind: int, layer: int):
        """Layer `layer`'s stage vector from the last persistent step: f32
        values for STAGE_XA / STAGE_XB / STAGE_Q; (int8 q[n], f32 d[n/32])
        for the Q8 vectors STAGE_O (attention output) and STAGE_H
        (silu(gate)*up).  Also returns the tags (high word halves)."""
        c = self.cfg
        n = {0: c["n_embd"], 1: c["n_embd"], 2: c["n_head"] * c["head_dim"],
             4: c["n_head"] * c["head_dim"], 5: c["n_ff"]}[kind]
        words = n if kind in (0, 1, 2) else n // 32 * 9
        p = self.lib.tf_model_stage_vector(self.h, kind, layer)
        if not p:
            raise capi.HipError("stage vectors are not kept (keep_stage_vectors before the step)")
        w = np.empty(words, np.uint64)
        torch.cuda.synchronize()
        capi.memcpy_d2h(w, p)
        lo = (w & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        tags = (w >> np.uint64(32)).astype(np.uint32)
        if kind in (0, 1, 2):
            return lo.view(np.float32), tags
        g = lo.reshape(-1, 9)
        q = np.ascontiguousarray(g[:, :8]).view(np.int8).reshape(-1)
        d = np.ascontiguousarray(g[:, 8]).view(np.float32)
        return (q, d), tags

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

    def prefill(self, tokens, pos0: int = 0) -> int:
        """Run the prompt `tokens` (positions pos0 ..) through the batched
        prefill forward; their K/V rows land in the cache and the argmax of
        the last token's logits is returned (the first generated token)."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        arr = (C.c_int * len(tokens))(*tokens.tolist())
        nxt = C.c_int()
        rc = self.lib.tf_model_prefill(self.h, arr, len(tokens), pos0, C.byref(nxt), self.stream)
        if rc != 0:
            raise capi.HipError(f"tf_model_prefill returned {rc}")
        return nxt.value

    def generate_prefilled(self, prompt, n_gen: int, use_graph: bool = True):
        """Greedy continuation of `prompt` with the prompt run through
        prefill(): the first token is prefill's argmax, the rest decode
        steps (forward.rs forward_greedy, then single-token decode)."""
        first = self.prefill(prompt, 0)
        if n_gen <= 1:
            return np.array([first][:n_gen], np.int32)
        rest = self.generate([first], n_gen - 1, pos0=len(prompt), use_graph=use_graph)
        return np.concatenate([[first], rest]).astype(np.int32)

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
