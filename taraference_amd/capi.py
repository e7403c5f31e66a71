"""ctypes binding of libtaraference_hip.so (the C ABI in include/taraference_hip.h).

torch is imported first so that the library resolves libamdhip64.so.7 to the
HIP runtime torch already loaded; device buffers and streams come from torch
and are handed to the library as raw pointers.  There is no fallback: if the
library is missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import torch  # noqa: F401  (must precede the library load: shared HIP runtime)

LIB_PATH = Path(__file__).resolve().parent / "libtaraference_hip.so"

_P = C.c_void_p
_I = C.c_int
_F = C.c_float

# name -> argument types (every function returns int, a hipError_t)
SIGNATURES: dict[str, list] = {
    "tf_quantize_q8": [_P, _P, _P, _I, _P],
    "tf_gemv_q4k_q8": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q4k_q8_splitk": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "tf_gemv_splitk_reduce": [_P, _P, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q4k_pair": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P],
    "tf_gemv_q4k_dual": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "tf_gemv_q4k_ffn": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "tf_gemv_q4k_ffn_f32": [_P, _P, _P, _P, _I, _I, _I, _P],
    "tf_gemv_q4k_qkv": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                        _P, _P, _P, _P],
    "tf_gemv_q6k_compact_q8": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q6k_down_splitk": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q6k_compact_q8_splitk": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "tf_gemv_q6k_f32": [_P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q8_0_q8": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q8_0_f32": [_P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q8_0_q8_splitk": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "tf_gemv_q8_0_f32_splitk": [_P, _P, _P, _I, _I, _I, _I, _P],
    "tf_gemv_q5_0_f32": [_P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q5_0_f32_splitk": [_P, _P, _P, _I, _I, _I, _I, _P],
    "tf_gemv_q5_0_qk": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P],
    "tf_gemv_q5_0_qkv": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P],
    "tf_gemv_q8_0_qkv": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P],
    "tf_q6k_compact_repack": [_P, _P, _I, _I, _I, _P],
    "tf_flash_decode_partial": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "tf_gemm_q4k_f32": [_P, _P, _P, _I, _I, _I, _I, _P],
    "tf_gemm_q6k_f32": [_P, _P, _P, _I, _I, _I, _I, _P],
    "tf_attn_prefill": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P],
    "tf_attn_prefill_d": [_P, _P, _P, _P, _I, _I, _I, _P, _I, _F, _P],
    "tf_flash_decode_partial_d": [_P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _F, _P],
    "tf_flash_decode_reduce": [_P, _P, _I, _I, _I, _I, _P],
    "tf_flash_decode_n_split": [_I, _I],
    "tf_gemv_q4k_flash_out": [_P, _P, _I, _I, _I, _P, _I, _I, _I, _P, _P, _P, _P],
    "tf_flash_decode": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _F, _P],
    "tf_flash_decode_noalloc": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _F, _P],
    "tf_gemv_q4k_f32": [_P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "tf_gemv_q4k_ffn_norm": [_P, _P, _P, _P, _F, _P, _I, _I, _I, _P],
    "tf_fused_norm_qkv_rope_kv": [_P, _P, _F, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I,
                                  _I, _P, _P, _P, _I, _P, _F, _P],
    "tf_gemv_q6k_compact_f32": [_P, _P, _P, _I, _I, _I, _I, _P],
    "tf_fused_qkv_rope_kv": [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                             _P, _P, _P, _I, _P, _F, _P],
    "tf_norm_quant": [_P, _P, _F, _P, _P, _P, _I, _P],
    "tf_flash_decode_reduce_q8": [_P, _P, _P, _P, _I, _I, _I, _P],
    "tf_gemv_q6k_q8_argmax": [_P, _P, _P, _P, _I, _I, _I, _P, _P],
    "tf_gemv_q6k_head_argmax": [_P, _P, _P, _F, _P, _I, _I, _I, _P, _P],
    "tf_argmax_key_finalize": [_P, _P, _P],
    "tf_embed_row": [_P, _I, _P, _I, _P, _I, _I, _P],
    "tf_rms_norm": [_P, _P, _P, _I, _F, _P],
    "tf_rope_neox": [_P, _I, _I, _I, _P, _F, _P],
    "tf_copy_kv_f16": [_P, _P, _I, _P, _I, _P],
    "tf_argmax": [_P, _I, _P, _P],
    "tf_q4k_block_dots": [_P, _P, _P, _P, _I, _I, _I, _P],
    "tf_decode_step_quantize_q8": [_P, _I, _I, _P, _P, _P],
    "tf_stream_read_probe": [_P, C.c_longlong, _P, _I, _I, _I, _P],
    "tf_q6k_block_dots": [_P, _I, _P, _P, _I, _I, _I, _P],
    "tf_version": [],
    "tf_exported_symbol_count": [],
}


class HipError(RuntimeError):
    pass


_lib = None


def load(path: Path | str | None = None) -> C.CDLL:
    """Load the in-tree HIP library (raises if it has not been built).  `path`
    names another build of the same library; only the first load counts."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path or LIB_PATH)
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build it with `python -m taraference_amd.build` "
            "(or __graft_entry__.build()); there is no non-HIP fallback")
    lib = C.CDLL(str(p))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = C.c_int
    lib.tf_exported_symbol.argtypes = [C.c_int]
    lib.tf_exported_symbol.restype = C.c_char_p
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    lib = load()
    return [lib.tf_exported_symbol(i).decode() for i in range(lib.tf_exported_symbol_count())]


def ptr(t) -> int | None:
    """Device (or host) address of a tensor; None for None."""
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(stream=None) -> int | None:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream or None


# Entry points bound elsewhere with their own argtypes (taraference_amd/model.py).
BOUND_ELSEWHERE = {"tf_model_create", "tf_model_destroy", "tf_model_forward",
                   "tf_model_generate", "tf_model_set_path", "tf_model_get_path",
                   "tf_model_logits", "tf_model_prefill", "tf_model_keep_stage_vectors",
                   "tf_model_stage_vector", "tf_model_q8_record",
                   "tf_model_k_cache", "tf_model_v_cache", "tf_exported_symbol",
                   # taraference_amd/gguf.py
                   "tf_gguf_open", "tf_gguf_close", "tf_gguf_version", "tf_gguf_data_offset",
                   "tf_gguf_file_size", "tf_gguf_n_tensors", "tf_gguf_tensor_at",
                   "tf_gguf_find_tensor", "tf_gguf_meta_type", "tf_gguf_meta_u32",
                   "tf_gguf_meta_u64", "tf_gguf_meta_f32", "tf_gguf_meta_str",
                   "tf_gguf_meta_bool", "tf_gguf_meta_i64", "tf_gguf_meta_f64",
                   "tf_gguf_meta_array", "tf_gguf_meta_array_str", "tf_gguf_meta_array_f64",
                   "tf_ggml_block_size", "tf_ggml_type_size", "tf_ggml_nbytes",
                   "tf_gguf_model_config"}


def call(name: str, *args) -> None:
    """Call C-ABI entry point `name`; raise HipError on a non-zero status.

    Only entry points with declared argument types may be called: without
    them ctypes would pass device pointers as 32-bit C ints."""
    if name not in SIGNATURES:
        raise KeyError(f"{name} has no declared argtypes in capi.SIGNATURES")
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise HipError(f"{name} returned hipError {rc}")


_hip = None


def memcpy_d2h(dst, src_ptr: int) -> None:
    """Blocking copy of dst.nbytes bytes from device address src_ptr into the
    numpy array dst (through the HIP runtime torch loaded)."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
    rc = _hip.hipMemcpy(dst.ctypes.data_as(C.c_void_p), C.c_void_p(src_ptr), dst.nbytes, 2)
    if rc != 0:
        raise HipError(f"hipMemcpy returned {rc}")
