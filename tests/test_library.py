"""The C-ABI library loads and exports every entry point include/trixium.h declares (no compute
call: this runs without a GPU)."""

import ctypes
import os
import re

import numpy as np

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
    fake = ctypes.c_void_p(256)
    for n, K, what in ((0, 256, b"x rows"), (9, 256, b"x rows"), (8, 19456, b"staged bytes")):
        rc = L.trx_gemv_ternary_exact_rows(fake, 5, 4, K, fake, n, 0, 0, fake, fake, None)
        assert rc == _lib.TRX_E_INVALID and what in L.trx_last_error(), (n, K, L.trx_last_error())
    rc = L.trx_gemv_ternary_exact_rows(fake, 5, 4, 256, ctypes.c_void_p(264), 2, 0, 0, fake, fake, None)
    assert rc == _lib.TRX_E_INVALID and b"16-byte aligned" in L.trx_last_error()
    pb, wb = ctypes.c_size_t(), ctypes.c_size_t()
    rc = L.trx_pack_geometry(7, 4, 256, ctypes.byref(pb), ctypes.byref(wb))
    assert rc == _lib.TRX_E_INVALID and b"not ternary" in L.trx_last_error()
    rc = L.trx_pack_geometry(5, 4, 200, ctypes.byref(pb), ctypes.byref(wb))
    assert rc == _lib.TRX_E_INVALID and b"multiple of 128" in L.trx_last_error()
    # The decode-state checkpoint and the KV ring refuse a missing model or an unknown request.
    assert L.trx_model_checkpoint(None, 0) == _lib.TRX_E_INVALID
    assert L.trx_model_checkpoint(fake, 2) == _lib.TRX_E_INVALID
    assert L.trx_model_set_kv_ring(None, 1, 4) == _lib.TRX_E_INVALID
    assert L.trx_model_set_kv_ring(fake, 2, 4) == _lib.TRX_E_INVALID
    assert L.trx_model_set_kv_ring(fake, 1, -1) == _lib.TRX_E_INVALID


def test_decoder_config_from_images(tiny_images):
    """The decoder's trx_model_config derived from the fixture images (host logic only)."""
    from trixium_amd import bons, layout as L
    from trixium_amd.model import config_from_header, make_config, rope_frequencies
    img = bons.BONSReader(tiny_images[("tiny-hybrid", True)])
    mc = config_from_header(img.header)
    c = make_config(mc, L.KIND_TERNARY5, L.KIND_F16, False, 0, L.KIND_TERNARY5, max_new=8)
    assert (c.n_layer, c.n_embd, c.vocab, c.max_ctx) == (4, 256, 1024, img.header["max_ctx"])
    assert c.layer_types[0] == 0b0111 and c.layer_types[1] == 0
    assert c.attn_gated == 1 and c.rope_dims == 16 and c.dn_num_v_heads == 8
    f = rope_frequencies(mc.rope_theta, 16)
    assert f.dtype == np.float32 and f[0] == 1.0 and np.all(np.diff(f) < 0)
