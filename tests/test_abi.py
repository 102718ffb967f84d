"""The C ABI library, without a GPU: it loads, exports every symbol that
include/mlk_hip.h declares, and rejects invalid arguments before any launch."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mlk_hip.h"
LIB = ROOT / "montlok.cpp_amd" / "montlok" / "rdt" / "lib" / "libmlk_hip.so"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int|size_t|mlk_status)\s+(mlk_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} missing: build with __graft_entry__.build()")
    return C.CDLL(str(LIB))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "mlk_rms_norm" in names and "mlk_mhc_prepare" in names
    assert len(names) >= 10


def test_library_exports_every_declared_symbol(lib):
    missing = [name for name in declared_symbols() if not hasattr(lib, name)]
    assert not missing, f"not exported: {missing}"


def test_python_module_binds_every_declared_symbol():
    from montlok import _C

    assert set(declared_symbols()) <= set(_C.exported_symbols())


def test_abi_version_and_last_error(lib):
    lib.mlk_abi_version.restype = C.c_int
    lib.mlk_last_error.restype = C.c_char_p
    assert lib.mlk_abi_version() == 1
    assert lib.mlk_last_error() == b""


def test_invalid_arguments_are_rejected_before_launch(lib):
    lib.mlk_last_error.restype = C.c_char_p
    f = lib.mlk_rms_norm
    f.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_double, C.c_int64, C.c_void_p,
                  C.c_void_p]
    f.restype = C.c_int
    assert f(None, 4, 10, 10, None, 1e-5, 3, None, None) == 1  # MLK_ERR_INVALID_ARGUMENT
    assert b"groups must divide" in lib.mlk_last_error()
    g = lib.mlk_mhc_prepare
    g.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_double,
                  C.c_void_p] + [C.c_void_p] * 6 + [C.c_int64, C.c_void_p, C.c_double] + [C.c_void_p] * 5
    g.restype = C.c_int
    assert g(None, 8, 4, 16, 16, 64, None, 1e-5, None, None, None, None, None, None, None, -1, None, 0.0, None, None,
             None, None, None) == 1
    assert b"sinkhorn_iters must be non-negative" in lib.mlk_last_error()
