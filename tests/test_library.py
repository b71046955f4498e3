"""The C-ABI library loads and exports every entry point include/trixium.h declares (no compute
call: this runs without a GPU)."""

import ctypes
import os
import re

from trixium_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    with open(os.path.join(ROOT, "include", "trixium.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int)\s+(trx_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "trx_gemv_ternary_exact" in names and "trx_last_error" in names
    assert len(names) >= 20


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(L, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert set(declared_symbols()) <= set(_lib.SIGNATURES), set(declared_symbols()) - set(_lib.SIGNATURES)


def test_errors_are_reported_without_a_device_call():
    L = _lib.lib()
    rc = L.trx_gemv_ternary_exact(None, 5, 4, 256, None, 0, 0, None, None, None)
    assert rc == _lib.TRX_E_INVALID
    assert b"null" in L.trx_last_error()
    rc = L.trx_gemv_ternary_f32(ctypes.c_void_p(16), 7, 4, 256, None, None, 1e-6, None, 0, None, None)
    assert rc == _lib.TRX_E_INVALID
