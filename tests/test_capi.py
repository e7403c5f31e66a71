"""C-ABI checks that need no GPU: the library loads, exports exactly the entry
points include/taraference_hip.h declares, does not link the oracle, and
rejects bad shapes with hipErrorInvalidValue before touching the device."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "taraference_hip.h"


def header_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^[A-Za-z][\w \*]*?\b(tf_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def capi():
    from taraference_amd import capi as c
    c.load()
    return c


def test_header_matches_exports(capi):
    hs = header_symbols()
    assert len(hs) >= 20
    assert sorted(capi.exported_symbols()) == hs
    lib = capi.load()
    for s in hs:
        assert hasattr(lib, s), s


def test_dynamic_symbols_present():
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "taraference_amd" /
                          "libtaraference_hip.so")], capture_output=True, text=True).stdout
    names = {l.split()[-1] for l in out.splitlines() if l.strip()}
    for s in header_symbols():
        assert s in names, s


def test_no_oracle_link():
    out = subprocess.run(["readelf", "-d", str(ROOT / "taraference_amd" /
                          "libtaraference_hip.so")], capture_output=True, text=True).stdout
    assert "oracle" not in out
    assert "libamdhip64" in out


def test_invalid_args_rejected(capi):
    lib = capi.load()
    INVALID = 1  # hipErrorInvalidValue
    assert lib.tf_quantize_q8(None, None, None, 64, None) == INVALID
    assert lib.tf_quantize_q8(8, 8, 8, 31, None) == INVALID          # K % 32 != 0
    assert lib.tf_gemv_q4k_q8(16, 16, 16, 16, 255, 4, 144, 0, None, 0, None, None) == INVALID
    assert lib.tf_gemv_q4k_q8(16, 16, 16, 16, 256, 4, 100, 0, None, 0, None, None) == INVALID
    assert lib.tf_gemv_q4k_q8(17, 16, 16, 16, 256, 4, 144, 0, None, 0, None, None) == INVALID
    assert lib.tf_gemv_q4k_q8(16, 16, 16, 16, 256, 4, 144, 1, None, 0, None, None) == INVALID
    assert lib.tf_gemv_q4k_q8(16, 16, 16, 16, 256, 4, 144, 0, None, 3, None, None) == INVALID
    assert lib.tf_gemv_q6k_compact_q8(16, 16, 16, 16, 256, 4, 210, 0, None, 0, None, None) == INVALID
    assert lib.tf_gemv_q4k_q8_splitk(16, 16, 16, 16, 2048, 4, 1152, 9, None) == INVALID
    assert lib.tf_flash_decode_partial(16, 16, 16, 16, 16, 3, 128, 10, 1, 8, 0.1, None) == INVALID
    assert lib.tf_flash_decode_partial(16, 16, 16, 16, 16, 2, 96, 10, 1, 8, 0.1, None) == INVALID
    assert lib.tf_flash_decode_partial(16, 16, 16, 16, 16, 2, 128, 10, 2, 8, 0.1, None) == INVALID
    assert lib.tf_flash_decode_reduce(16, 16, 16, 128, 0, 1, None) == INVALID
    assert lib.tf_norm_quant(16, 16, 1e-6, 16, 16, 16, 96, None) == INVALID   # n % 128
    assert lib.tf_norm_quant(16, 16, 1e-6, 16, 16, 16, 8320, None) == INVALID  # n > 8192
    # prefill GEMMs: K not a multiple of 4, or a column shorter than its blocks
    assert lib.tf_gemm_q4k_f32(16, 16, 16, 512 + 2, 16, 2 * 144, 1, None) == INVALID
    assert lib.tf_gemm_q6k_f32(16, 16, 16, 512, 16, 2 * 210 - 2, 1, None) == INVALID
    assert lib.tf_version() >= 100


def test_every_export_has_argtypes(capi):
    """A C-ABI function called without declared argtypes gets its pointer
    arguments truncated to 32-bit C ints; every export must be declared."""
    declared = set(capi.SIGNATURES) | capi.BOUND_ELSEWHERE
    missing = [s for s in header_symbols() if s not in declared]
    assert not missing, missing
    for name, args in capi.SIGNATURES.items():
        assert name in header_symbols(), name
    import ctypes
    lib = capi.load()
    assert lib.tf_gemv_q6k_compact_f32.argtypes[0] is ctypes.c_void_p


def header_param_counts():
    text = HEADER.read_text()
    out = {}
    for m in re.finditer(r"^[A-Za-z][\w \*]*?\b(tf_\w+)\s*\(([^;]*?)\)\s*;", text, re.M | re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_argtypes_match_header_arity(capi):
    counts = header_param_counts()
    for name, args in capi.SIGNATURES.items():
        assert counts[name] == len(args), (name, counts[name], len(args))
