"""Python handle on the GGUF reader (tf_gguf_* in include/taraference_hip.h,
the C++ restatement of crates/gguf/src/reader.rs).

The file is memory-mapped by the library; tensor bytes come back as numpy
views of the mapping (valid while the GgufFile is open).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import capi

ERR_NOT_FOUND = 1009
ERR_TYPE = 1010

# value.rs:8-23
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)

# ggml type ids (types.rs:7-36) used by the decode path
GGML_F32, GGML_F16, GGML_Q4_K, GGML_Q6_K = 0, 1, 12, 14


class GgufError(RuntimeError):
    def __init__(self, what: str, code: int):
        super().__init__(f"{what}: GGUF error {code}")
        self.code = code


class TfGgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("n_dims", C.c_int),
                ("dims", C.c_uint64 * 4), ("offset", C.c_uint64), ("nbytes", C.c_uint64),
                ("data", C.c_void_p)]


class TfModelConfig(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("n_embd", C.c_int), ("n_ff", C.c_int),
                ("n_head", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
                ("n_vocab", C.c_int), ("max_seq", C.c_int), ("rope_theta", C.c_float),
                ("rms_eps", C.c_float)]


_bound = False


def _bind(lib):
    global _bound
    if _bound:
        return
    P, H = C.c_void_p, C.c_void_p
    sigs = {
        "tf_gguf_open": ([C.c_char_p, C.POINTER(C.c_void_p)], C.c_int),
        "tf_gguf_close": ([H], None),
        "tf_gguf_version": ([H], C.c_uint32),
        "tf_gguf_data_offset": ([H], C.c_uint64),
        "tf_gguf_file_size": ([H], C.c_uint64),
        "tf_gguf_n_tensors": ([H], C.c_int64),
        "tf_gguf_tensor_at": ([H, C.c_int64, C.POINTER(TfGgufTensor)], C.c_int),
        "tf_gguf_find_tensor": ([H, C.c_char_p, C.POINTER(TfGgufTensor)], C.c_int),
        "tf_gguf_meta_type": ([H, C.c_char_p], C.c_int),
        "tf_gguf_meta_u32": ([H, C.c_char_p, C.POINTER(C.c_uint32)], C.c_int),
        "tf_gguf_meta_u64": ([H, C.c_char_p, C.POINTER(C.c_uint64)], C.c_int),
        "tf_gguf_meta_f32": ([H, C.c_char_p, C.POINTER(C.c_float)], C.c_int),
        "tf_gguf_meta_str": ([H, C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)],
                             C.c_int),
        "tf_gguf_meta_bool": ([H, C.c_char_p, C.POINTER(C.c_int)], C.c_int),
        "tf_gguf_meta_i64": ([H, C.c_char_p, C.POINTER(C.c_int64)], C.c_int),
        "tf_gguf_meta_f64": ([H, C.c_char_p, C.POINTER(C.c_double)], C.c_int),
        "tf_gguf_meta_array": ([H, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_uint64)],
                               C.c_int),
        "tf_gguf_meta_array_str": ([H, C.c_char_p, C.c_uint64, C.POINTER(C.c_void_p),
                                    C.POINTER(C.c_uint64)], C.c_int),
        "tf_gguf_meta_array_f64": ([H, C.c_char_p, C.c_uint64, C.POINTER(C.c_double)], C.c_int),
        "tf_ggml_block_size": ([C.c_int], C.c_int),
        "tf_ggml_type_size": ([C.c_int], C.c_int),
        "tf_ggml_nbytes": ([C.c_int, C.c_uint64], C.c_uint64),
        "tf_gguf_model_config": ([H, C.c_int, C.POINTER(TfModelConfig)], C.c_int),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _bound = True


def lib():
    L = capi.load()
    _bind(L)
    return L


def ggml_block_size(t: int) -> int:
    return lib().tf_ggml_block_size(t)


def ggml_type_size(t: int) -> int:
    return lib().tf_ggml_type_size(t)


def ggml_nbytes(t: int, n: int) -> int:
    return lib().tf_ggml_nbytes(t, n)


class GgufFile:
    """reader.rs GgufFile: open(), metadata accessors, tensor(name), tensor_data()."""

    def __init__(self, path):
        self.lib = lib()
        h = C.c_void_p()
        rc = self.lib.tf_gguf_open(str(path).encode(), C.byref(h))
        if rc != 0:
            raise GgufError(f"open {path}", rc)
        self.h = h
        self.path = str(path)

    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.tf_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    # ------------------------------------------------------------ header
    @property
    def version(self) -> int:
        return self.lib.tf_gguf_version(self.h)

    @property
    def data_offset(self) -> int:
        return self.lib.tf_gguf_data_offset(self.h)

    @property
    def file_size(self) -> int:
        return self.lib.tf_gguf_file_size(self.h)

    # ---------------------------------------------------------- metadata
    def meta_type(self, key: str) -> int:
        return self.lib.tf_gguf_meta_type(self.h, key.encode())

    def _get(self, fn, ctype, key):
        v = ctype()
        rc = getattr(self.lib, fn)(self.h, key.encode(), C.byref(v))
        if rc in (ERR_NOT_FOUND, ERR_TYPE):
            return None
        if rc != 0:
            raise GgufError(f"{fn} {key}", rc)
        return v.value

    def meta_u32(self, key):
        return self._get("tf_gguf_meta_u32", C.c_uint32, key)

    def meta_u64(self, key):
        return self._get("tf_gguf_meta_u64", C.c_uint64, key)

    def meta_f32(self, key):
        return self._get("tf_gguf_meta_f32", C.c_float, key)

    def meta_i64(self, key):
        return self._get("tf_gguf_meta_i64", C.c_int64, key)

    def meta_f64(self, key):
        return self._get("tf_gguf_meta_f64", C.c_double, key)

    def meta_bool(self, key):
        v = self._get("tf_gguf_meta_bool", C.c_int, key)
        return None if v is None else bool(v)

    def meta_str(self, key):
        s, n = C.c_void_p(), C.c_uint64()
        rc = self.lib.tf_gguf_meta_str(self.h, key.encode(), C.byref(s), C.byref(n))
        if rc in (ERR_NOT_FOUND, ERR_TYPE):
            return None
        if rc != 0:
            raise GgufError(f"meta_str {key}", rc)
        return C.string_at(s.value, n.value).decode() if n.value else ""

    def meta_array(self, key):
        """(item_type, list of items) for an array of numbers or strings."""
        it, n = C.c_int(), C.c_uint64()
        rc = self.lib.tf_gguf_meta_array(self.h, key.encode(), C.byref(it), C.byref(n))
        if rc in (ERR_NOT_FOUND, ERR_TYPE):
            return None
        items = []
        for i in range(n.value):
            if it.value == STRING:
                s, ln = C.c_void_p(), C.c_uint64()
                self.lib.tf_gguf_meta_array_str(self.h, key.encode(), i, C.byref(s), C.byref(ln))
                items.append(C.string_at(s.value, ln.value).decode() if ln.value else "")
            else:
                d = C.c_double()
                rc = self.lib.tf_gguf_meta_array_f64(self.h, key.encode(), i, C.byref(d))
                items.append(None if rc else d.value)
        return it.value, items

    def architecture(self):
        return self.meta_str("general.architecture")

    # ----------------------------------------------------------- tensors
    def n_tensors(self) -> int:
        return self.lib.tf_gguf_n_tensors(self.h)

    def tensor(self, name: str) -> TfGgufTensor | None:
        t = TfGgufTensor()
        rc = self.lib.tf_gguf_find_tensor(self.h, name.encode(), C.byref(t))
        if rc == ERR_NOT_FOUND:
            return None
        if rc != 0:
            raise GgufError(f"tensor {name}", rc)
        return t

    def tensors(self) -> list[TfGgufTensor]:
        out = []
        for i in range(self.n_tensors()):
            t = TfGgufTensor()
            rc = self.lib.tf_gguf_tensor_at(self.h, i, C.byref(t))
            if rc != 0:
                raise GgufError(f"tensor_at {i}", rc)
            out.append(t)
        return out

    def tensor_data(self, t: TfGgufTensor) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view of the mapping."""
        if t.nbytes == 0:
            return np.zeros(0, np.uint8)
        buf = (C.c_uint8 * t.nbytes).from_address(t.data)
        a = np.ctypeslib.as_array(buf)
        a.flags.writeable = False
        return a

    def model_config(self, max_seq: int) -> dict:
        cfg = TfModelConfig()
        rc = self.lib.tf_gguf_model_config(self.h, max_seq, C.byref(cfg))
        if rc != 0:
            raise GgufError("model config", rc)
        return {f: getattr(cfg, f) for f, _ in TfModelConfig._fields_}
