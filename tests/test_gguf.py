"""The GGUF reader (tf_gguf_*, crates/gguf/src/reader.rs semantics) on files
written by tests/_gguf_write.py: every metadata value type, tensors of the
decode path's types, v2 and v3 headers, the data-section alignment, the
value conversions of value.rs:72-106, the ggml type table, every error the
reference reports, and the dense model configuration of config.rs:107-175.
No GPU: the reader is host code."""
import struct

import numpy as np
import pytest

import _gguf_write as W
from taraference_amd import gguf as G

ERR = dict(IO=1001, MAGIC=1002, VERSION=1003, EOF=1004, MALFORMED=1005, TENSOR_TYPE=1006,
           VALUE_TYPE=1007, UTF8=1008)


def _meta_all():
    return [
        ("t.u8", W.U8, 200), ("t.i8", W.I8, -100), ("t.u16", W.U16, 60000),
        ("t.i16", W.I16, -30000), ("t.u32", W.U32, 4000000000), ("t.i32", W.I32, -7),
        ("t.i32pos", W.I32, 12345), ("t.f32", W.F32, 1.5), ("t.bool", W.BOOL, True),
        ("t.str", W.STRING, "héllo · wörld"), ("t.u64", W.U64, 1 << 40),
        ("t.u64small", W.U64, 77), ("t.i64", W.I64, -(1 << 40)), ("t.i64pos", W.I64, 99),
        ("t.f64", W.F64, 0.1),
        ("t.arr_u32", W.ARRAY, (W.U32, [1, 2, 3])),
        ("t.arr_str", W.ARRAY, (W.STRING, ["a", "", "ccc"])),
        ("t.arr_f32", W.ARRAY, (W.F32, [0.5, -2.0])),
        ("t.arr_arr", W.ARRAY, (W.ARRAY, [(W.U8, [1, 2]), (W.U8, [])])),
        ("t.empty", W.STRING, ""),
    ]


def _tensors(rng):
    q4 = rng.integers(0, 256, (3, 2 * 144), dtype=np.uint8)    # Q4_K [512, 3]
    q6 = rng.integers(0, 256, (2, 210), dtype=np.uint8)        # Q6_K [256, 2]
    f32 = rng.standard_normal(10).astype(np.float32)
    f16 = rng.standard_normal((2, 3)).astype(np.float16)
    q8 = rng.integers(0, 256, (4, 34), dtype=np.uint8)         # Q8_0 [32, 2, 2]
    return [
        ("w.q4", [512, 3], 12, q4.tobytes()),
        ("w.q6", [256, 2], 14, q6.tobytes()),
        ("v.f32", [10], 0, f32.tobytes()),
        ("v.f16", [3, 2], 1, f16.tobytes()),
        ("w.q8", [32, 2, 2], 8, q8.tobytes()),
        ("s.scalar", [], 0, np.float32(3.25).tobytes()),
    ]


@pytest.mark.parametrize("version,align", [(3, None), (2, None), (3, 64), (3, 1)])
def test_roundtrip(tmp_path, version, align):
    rng = np.random.default_rng(1)
    meta = _meta_all()
    if align is not None:
        meta = [("general.alignment", W.U32, align)] + meta
    tens = _tensors(rng)
    p = tmp_path / "a.gguf"
    W.write(p, meta, tens, version=version)
    raw = p.read_bytes()
    with G.GgufFile(p) as f:
        assert f.version == version
        assert f.file_size == len(raw)
        a = 32 if align is None else align
        assert f.data_offset % a == 0
        assert f.n_tensors() == len(tens)
        for (name, dims, ty, data), t in zip(tens, f.tensors()):
            assert t.name.decode() == name and t.type == ty and t.n_dims == len(dims)
            assert list(t.dims[:t.n_dims]) == dims and list(t.dims[t.n_dims:]) == [1] * (4 - len(dims))
            assert t.nbytes == len(data)
            got = f.tensor_data(t)
            assert got.tobytes() == data
            assert raw[f.data_offset + t.offset:f.data_offset + t.offset + t.nbytes] == data
        assert f.tensor("w.q6").type == 14 and f.tensor("nope") is None
        # metadata, type ids and the value.rs conversions
        assert f.meta_type("t.str") == W.STRING and f.meta_type("missing") == -1
        assert f.meta_str("t.str") == "héllo · wörld" and f.meta_str("t.empty") == ""
        assert f.meta_u32("t.u8") == 200 and f.meta_u32("t.u16") == 60000
        assert f.meta_u32("t.u32") == 4000000000
        assert f.meta_u32("t.u64small") == 77 and f.meta_u32("t.u64") is None
        assert f.meta_u32("t.i32pos") == 12345 and f.meta_u32("t.i32") is None
        assert f.meta_u32("t.i64pos") is None            # as_u32 takes no I64
        assert f.meta_u64("t.u64") == 1 << 40 and f.meta_u64("t.i64pos") == 99
        assert f.meta_u64("t.i64") is None and f.meta_u64("t.i8") is None
        assert f.meta_f32("t.f32") == 1.5 and f.meta_f32("t.f64") == np.float32(0.1)
        assert f.meta_f32("t.u32") is None
        assert f.meta_bool("t.bool") is True and f.meta_str("t.u8") is None
        assert f.meta_i64("t.i64") == -(1 << 40) and f.meta_i64("t.i8") == -100
        assert f.meta_f64("t.f64") == 0.1
        assert f.meta_array("t.arr_u32") == (W.U32, [1.0, 2.0, 3.0])
        assert f.meta_array("t.arr_str") == (W.STRING, ["a", "", "ccc"])
        assert f.meta_array("t.arr_f32") == (W.F32, [0.5, -2.0])
        it, items = f.meta_array("t.arr_arr")
        assert it == W.ARRAY and len(items) == 2


def test_alignment_zero_and_repeated_keys(tmp_path):
    # alignment 0: the data section starts right after the header
    meta = [("general.alignment", W.U64, 0), ("k", W.U32, 1), ("k", W.U32, 2)]
    tens = [("x", [3], 0, np.arange(3, dtype=np.float32).tobytes())]
    p = tmp_path / "z.gguf"
    raw = W.build(meta, tens, alignment=0)
    p.write_bytes(raw)
    with G.GgufFile(p) as f:
        assert f.data_offset == len(raw) - 12
        assert f.meta_u32("k") == 2                      # the last value wins (HashMap insert)
        assert np.array_equal(f.tensor_data(f.tensor("x")).view(np.float32), [0, 1, 2])


def _open_code(path):
    try:
        G.GgufFile(path).close()
    except G.GgufError as e:
        return e.code
    return 0


def test_errors(tmp_path):
    good = W.build([("a", W.U32, 1)], [("x", [4], 0, b"\0" * 16)])
    cases = {}
    cases["magic"] = b"GGUG" + good[4:]
    cases["v1"] = good[:4] + struct.pack("<I", 1) + good[8:]
    cases["v4"] = good[:4] + struct.pack("<I", 4) + good[8:]
    cases["short"] = good[:20]
    cases["nodata"] = good[:-8]                                   # tensor past EOF
    cases["counts"] = struct.pack("<IIQQ", 0x46554747, 3, 2_000_000, 0)
    cases["ndims"] = W.build([], [("x", [1, 1, 1, 1, 1], 0, b"\0" * 4)])
    cases["ttype"] = W.build([], [("x", [4], 4, b"\0" * 16)])      # ids 4, 5 were removed
    vt = W.build([("a", W.U32, 1)], [])
    cases["vtype"] = vt.replace(struct.pack("<Q", 1) + b"a" + struct.pack("<I", 4),
                                struct.pack("<Q", 1) + b"a" + struct.pack("<I", 13))
    cases["utf8"] = W.build([(b"\xff\xfe", W.U32, 1)], [])
    cases["strlen"] = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1 << 30)
    cases["arrlen"] = (struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + W._string("a") +
                       struct.pack("<IIQ", W.ARRAY, W.U8, 20_000_000))
    want = dict(magic="MAGIC", v1="VERSION", v4="VERSION", short="EOF", nodata="MALFORMED",
                counts="MALFORMED", ndims="MALFORMED", ttype="TENSOR_TYPE", vtype="VALUE_TYPE",
                utf8="UTF8", strlen="MALFORMED", arrlen="MALFORMED")
    for k, data in cases.items():
        p = tmp_path / f"{k}.gguf"
        p.write_bytes(data)
        assert _open_code(p) == ERR[want[k]], k
    assert _open_code(tmp_path / "does-not-exist.gguf") == ERR["IO"]
    (tmp_path / "ok.gguf").write_bytes(good)
    assert _open_code(tmp_path / "ok.gguf") == 0


def test_type_table():
    """Sizes from the GGML block layouts themselves (ggml's block structs):
    a 32-value block is its f16 scale(s) plus the packed quants, a 256-value
    super-block its scales, quants and f16/f32 factors."""
    derived = {
        0: (1, 4), 1: (1, 2), 30: (1, 2), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8),
        28: (1, 8),
        2: (32, 2 + 16),                 # Q4_0: d, 32 nibbles
        3: (32, 2 + 2 + 16),             # Q4_1: d, m, nibbles
        6: (32, 2 + 4 + 16),             # Q5_0: d, 32 high bits, nibbles
        7: (32, 2 + 2 + 4 + 16),         # Q5_1
        8: (32, 2 + 32),                 # Q8_0: d, 32 int8
        9: (32, 2 + 2 + 32),             # Q8_1: d, s, 32 int8
        10: (256, 16 + 64 + 2 + 2),      # Q2_K: scales, 2-bit quants, d, dmin
        11: (256, 32 + 64 + 12 + 2),     # Q3_K: hmask, quants, scales, d
        12: (256, 2 + 2 + 12 + 128),     # Q4_K
        13: (256, 2 + 2 + 12 + 32 + 128),  # Q5_K
        14: (256, 128 + 64 + 16 + 2),    # Q6_K
        15: (256, 4 + 256 + 2 * 16),     # Q8_K: f32 d, int8, int16 block sums
    }
    for t, (blk, sz) in derived.items():
        assert (G.ggml_block_size(t), G.ggml_type_size(t)) == (blk, sz), t
    for t in (4, 5, 31, 99, -1):
        assert G.ggml_type_size(t) == 0 and G.ggml_nbytes(t, 256) == 0
    assert G.ggml_nbytes(12, 2048) == 8 * 144 and G.ggml_nbytes(12, 257) == 2 * 144
    assert G.ggml_nbytes(8, 33) == 2 * 34 and G.ggml_nbytes(0, 7) == 28


def _cfg_file(tmp_path, meta, tensors=()):
    p = tmp_path / "cfg.gguf"
    W.write(p, meta, list(tensors))
    return G.GgufFile(p)


def test_model_config(tmp_path):
    base = [("general.architecture", W.STRING, "qwen2"),
            ("qwen2.embedding_length", W.U32, 2048), ("qwen2.block_count", W.U32, 36),
            ("qwen2.attention.head_count", W.U32, 16),
            ("qwen2.attention.head_count_kv", W.U32, 2),
            ("qwen2.feed_forward_length", W.U32, 11008), ("qwen2.vocab_size", W.U32, 151936),
            ("qwen2.rope.freq_base", W.F32, 1000000.0),
            ("qwen2.attention.layer_norm_rms_epsilon", W.F32, 1e-6)]
    with _cfg_file(tmp_path, base) as f:
        c = f.model_config(4096)
    assert c == dict(n_layer=36, n_embd=2048, n_ff=11008, n_head=16, n_kv=2, head_dim=128,
                     n_vocab=151936, max_seq=4096, rope_theta=1e6,
                     rms_eps=float(np.float32(1e-6)))
    # defaults: kv heads = heads, head_dim = n_embd / heads, vocab from
    # token_embd.weight dims[1], theta 1e4 for llama (llama3 maps to llama)
    m = [("general.architecture", W.STRING, "llama3"), ("llama.embedding_length", W.U64, 512),
         ("llama.block_count", W.I32, 2), ("llama.attention.head_count", W.U32, 4),
         ("llama.feed_forward_length", W.U32, 768)]
    emb = ("token_embd.weight", [512, 1000], 12, b"\0" * (2 * 144 * 1000))
    with _cfg_file(tmp_path, m, [emb]) as f:
        c = f.model_config(64)
    assert (c["n_kv"], c["head_dim"], c["n_vocab"], c["rope_theta"], c["rms_eps"]) == \
        (4, 128, 1000, 10000.0, float(np.float32(1e-6)))
    assert c["n_embd"] == 512 and c["n_layer"] == 2
    with _cfg_file(tmp_path, [x for x in base if "freq_base" not in x[0]]) as f:
        assert f.model_config(8)["rope_theta"] == 1e6
    for drop in ("qwen2.block_count", "general.architecture"):
        with _cfg_file(tmp_path, [x for x in base if x[0] != drop]) as f:
            with pytest.raises(G.GgufError):
                f.model_config(8)
    with _cfg_file(tmp_path, base + [("qwen2.attention.key_length", W.U32, 128),
                                     ("qwen2.attention.value_length", W.U32, 64)]) as f:
        with pytest.raises(G.GgufError):
            f.model_config(8)
