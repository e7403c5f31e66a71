"""A GGUF writer for test fixtures (the GGUF v2/v3 container as the
reference's reader parses it: crates/gguf/src/reader.rs:29-169,
value.rs:187-287).  Little-endian throughout:

  u32 magic "GGUF" | u32 version | u64 n_tensors | u64 n_kv
  n_kv x (string key, u32 value type, value)
  n_tensors x (string name, u32 n_dims, u64 dims[n_dims], u32 ggml type,
               u64 offset relative to the data section)
  padding to general.alignment (32 if absent) | tensor data

string = u64 length + bytes; array = u32 item type + u64 count + items.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}

# ggml (block elements, bytes per block) of the types the fixtures use
TYPES = {0: (1, 4), 1: (1, 2), 6: (32, 22), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def _string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(ty: int, v) -> bytes:
    if ty == STRING:
        return _string(v)
    if ty == ARRAY:
        item_ty, items = v
        out = struct.pack("<IQ", item_ty, len(items))
        for it in items:
            out += _value(item_ty, it)
        return out
    if ty == BOOL:
        return struct.pack("<B", 1 if v else 0)
    return struct.pack(_FMT[ty], v)


def nbytes(ggml_type: int, n: int) -> int:
    blk, sz = TYPES[ggml_type]
    return (n + blk - 1) // blk * sz


def build(meta, tensors, version: int = 3, alignment: int | None = None,
          data_pad: int = 0) -> bytes:
    """meta: [(key, value type, value)]; tensors: [(name, dims, ggml type,
    bytes)].  Tensor data is laid out in order, each start aligned; the
    alignment is general.alignment from meta when present (else 32) unless
    given.  data_pad extra bytes are appended at the end."""
    if alignment is None:
        alignment = 32
        for k, ty, v in meta:
            if k == "general.alignment":
                alignment = v
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(meta))
    for k, ty, v in meta:
        head += _string(k) + struct.pack("<I", ty) + _value(ty, v)
    offsets, off = [], 0
    for name, dims, ty, data in tensors:
        if alignment:
            off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += len(data)
    for (name, dims, ty, data), o in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, o)
    start = len(head)
    if alignment:
        start = (start + alignment - 1) // alignment * alignment
    out = bytearray(head + b"\0" * (start - len(head)))
    for (name, dims, ty, data), o in zip(tensors, offsets):
        out += b"\0" * (start + o - len(out))
        out += bytes(data)
    out += b"\0" * data_pad
    return bytes(out)


def write(path, meta, tensors, **kw) -> None:
    with open(path, "wb") as f:
        f.write(build(meta, tensors, **kw))


def model_tensors(cfg: dict, layers, embedding, output=None, output_norm=None,
                  arch: str = "qwen2"):
    """(meta, tensors) of a dense decoder in the reference's GGUF names
    (cuda/load.rs:280-420) from synth.qwen_layer() dicts: matrices are
    [n_cols, col_bytes] byte arrays stored with dims [n_rows, n_cols]."""
    meta = model_meta(cfg, arch)
    c = cfg
    qd, kvd = c["n_head"] * c["head_dim"], c["n_kv"] * c["head_dim"]
    t = []
    return _model_tensor_list(cfg, layers, embedding, output, output_norm, meta, t, qd, kvd)


def model_meta(cfg: dict, arch: str = "qwen2"):
    """The metadata of a dense decoder (config.rs:107-175 keys)."""
    c = cfg
    meta = [
        ("general.architecture", STRING, arch),
        ("general.name", STRING, "synthetic"),
        (f"{arch}.embedding_length", U32, c["n_embd"]),
        (f"{arch}.block_count", U32, c["n_layer"]),
        (f"{arch}.attention.head_count", U32, c["n_head"]),
        (f"{arch}.attention.head_count_kv", U32, c["n_kv"]),
        (f"{arch}.feed_forward_length", U32, c["n_ff"]),
        (f"{arch}.context_length", U32, 4096),
        (f"{arch}.rope.freq_base", F32, c["rope_theta"]),
        (f"{arch}.attention.layer_norm_rms_epsilon", F32, c["rms_eps"]),
    ]
    return meta


def _model_tensor_list(cfg, layers, embedding, output, output_norm, meta, t, qd, kvd):
    c = cfg

    def mat(name, wm, ty, n_rows):
        w, cb = wm[0], wm[1]
        assert cb == nbytes(ty, n_rows)
        t.append((name, [n_rows, w.shape[0]], ty, np.ascontiguousarray(w).tobytes()))

    def vec(name, v):
        t.append((name, [len(v)], 0, np.asarray(v, np.float32).tobytes()))

    mat("token_embd.weight", embedding, 14, c["n_embd"])
    vec("output_norm.weight", np.ones(c["n_embd"], np.float32) if output_norm is None
        else output_norm)
    if output is not None:
        mat("output.weight", output, 14, c["n_embd"])
    for i, L in enumerate(layers):
        p = f"blk.{i}"
        vec(f"{p}.attn_norm.weight", L["attn_norm"])
        vec(f"{p}.ffn_norm.weight", L["ffn_norm"])
        mat(f"{p}.attn_q.weight", L["wq"], 12, c["n_embd"])
        mat(f"{p}.attn_k.weight", L["wk"], 12, c["n_embd"])
        mat(f"{p}.attn_v.weight", L["wv"], 14, c["n_embd"])
        for k, n in (("bq", qd), ("bk", kvd), ("bv", kvd)):
            if L.get(k) is not None:
                assert len(L[k]) == n
                vec(f"{p}.attn_{k[1]}.bias", L[k])
        mat(f"{p}.attn_output.weight", L["wo"], 12, qd)
        mat(f"{p}.ffn_gate.weight", L["gate"], 12, c["n_embd"])
        mat(f"{p}.ffn_up.weight", L["up"], 12, c["n_embd"])
        mat(f"{p}.ffn_down.weight", L["down"], 14 if L["down_q6k"] else 12, c["n_ff"])
    return meta, t
