"""ctypes binding of libtrixium_hip.so (the C ABI declared in include/trixium.h).

The library is built in-tree (trixium_amd/libtrixium_hip.so). There is no CPU fallback: every
compute entry point of this package goes through the HIP library, and loading fails loudly when
it is missing.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtrixium_hip.so")

TRX_OK, TRX_E_INVALID, TRX_E_HIP, TRX_E_OVERFLOW, TRX_E_NOMEM, TRX_E_STATE = 0, -1, -2, -3, -4, -5
EPI_STORE, EPI_RESID, EPI_SWIGLU = 0, 1, 2

_vp, _i, _u64, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_float, ctypes.c_size_t
_ip = ctypes.POINTER(ctypes.c_int)
_fp = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)


class ModelConfig(ctypes.Structure):
    """trx_model_config of include/trixium.h."""
    _fields_ = [(n, ctypes.c_int) for n in ("n_layer", "n_embd", "n_head", "n_kv_head", "head_dim",
                                            "ffn_dim", "vocab", "max_ctx")] + [
        ("rms_eps", ctypes.c_float), ("rope_dims", ctypes.c_int), ("attn_gated", ctypes.c_int)] + [
        (n, ctypes.c_int) for n in ("dn_num_v_heads", "dn_num_k_heads", "dn_k_head_dim",
                                    "dn_v_head_dim", "dn_conv_kernel")] + [
        ("layer_types", ctypes.c_uint64 * 2)] + [
        (n, ctypes.c_int) for n in ("weight_kind", "head_kind", "head_tied", "emb_mode", "emb_kind",
                                    "max_new", "packed_ops")] + [
        ("hadamard_block", ctypes.c_int), ("hadamard_scale", ctypes.c_float),
        ("hadamard_widths", ctypes.c_int * 4), ("rope_table", ctypes.c_int), ("prefill_chunk", ctypes.c_int),
        ("table_free_ops", ctypes.c_int)]


_mcp = ctypes.POINTER(ModelConfig)

# name -> argtypes (restype is int unless listed in _RESTYPES)
class PartialSums(ctypes.Structure):
    """trx_partial_sums (include/trixium.h): split-K partial sums handed between packed GEMVs."""
    _fields_ = [("out", ctypes.c_void_p), ("out_ss", ctypes.c_void_p), ("in_", ctypes.c_void_p),
                ("in_ss", ctypes.c_void_p), ("resid", ctypes.c_void_p), ("S", ctypes.c_int),
                ("rows_p", ctypes.c_int), ("F", ctypes.c_int), ("in_K", ctypes.c_int),
                ("act", ctypes.c_void_p)]


SIGNATURES = {
    "trx_last_error": [],
    "trx_version": [],
    "trx_device_count": [_ip],
    "trx_set_device": [_i],
    "trx_device_name": [ctypes.c_char_p, _i],
    "trx_malloc": [ctypes.POINTER(_vp), _sz],
    "trx_free": [_vp],
    "trx_memcpy_h2d": [_vp, _vp, _sz, _vp],
    "trx_memcpy_d2h": [_vp, _vp, _sz, _vp],
    "trx_memcpy_d2d": [_vp, _vp, _sz, _vp],
    "trx_memset_d8": [_vp, _i, _sz, _vp],
    "trx_stream_create": [ctypes.POINTER(_vp)],
    "trx_stream_destroy": [_vp],
    "trx_stream_sync": [_vp],
    "trx_event_create": [ctypes.POINTER(_vp)],
    "trx_event_destroy": [_vp],
    "trx_event_record": [_vp, _vp],
    "trx_event_elapsed_ms": [_vp, _vp, _fp],
    "trx_gemv_ternary_exact": [_vp, _i, _i, _i, _vp, _i, _i, _vp, _vp, _vp],
    "trx_gemv_ternary_exact_rows": [_vp, _i, _i, _i, _vp, _i, _i, _i, _vp, _vp, _vp],
    "trx_gemv_ternary_groupsums": [_vp, _i, _i, _i, _vp, _vp, _vp],
    "trx_quantize_f_pow2": [_vp, _i, _vp, _vp, _vp],
    "trx_gemv_quantized_geometry": [_i, _i, ctypes.POINTER(_sz)],
    "trx_gemv_ternary_quantized": [_vp, _i, _i, _i, _vp, _i, _i, _vp, _vp, _vp, _vp],
    "trx_gemv_ternary_f32": [_vp, _i, _i, _i, _vp, _vp, _f, _vp, _i, _vp, _vp],
    "trx_pack_geometry": [_i, _i, _i, ctypes.POINTER(_sz), ctypes.POINTER(_sz)],
    "trx_pack_ternary": [_vp, _i, _i, _i, _i, _vp, _vp],
    "trx_gemv_packed_f32": [_vp, _i, _i, _i, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp],
    "trx_gemv_packed_f32_noalloc": [_vp, _i, _i, _i, _vp, _vp, _f, _vp, _i, _vp, _vp],
    "trx_pack_partials_geometry": [_i, _i, _i, _ip, _ip, _ip],
    "trx_pack_batched_geometry": [_i, _i, _i, _i, ctypes.POINTER(_sz)],
    "trx_gemv_packed_batched_f32": [_vp, _sz, _i, _i, _i, _i, _i, _vp, _i, _vp, _i, _vp, _vp],
    "trx_gemv_packed_parts_f32": [_vp, _i, _i, _i, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp, _vp],
    "trx_gemv_set_variant": [_i],
    "trx_model_create": [_mcp, _fp, ctypes.POINTER(_vp)],
    "trx_model_destroy": [_vp],
    "trx_model_set_tensor": [_vp, _i, _i, _vp, _sz],
    "trx_model_set_sampling": [_vp, ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_uint32, _i],
    "trx_model_synthesize": [_vp, ctypes.c_uint32, _fp],
    "trx_model_reset": [_vp],
    "trx_model_checkpoint": [_vp, _i],
    "trx_model_set_kv_ring": [_vp, _i, _i],
    "trx_model_set_prompt": [_vp, _ip, _i, _i],
    "trx_model_step": [_vp, _i, _i],
    "trx_model_prefill": [_vp, _i, _i],
    "trx_gemm_ternary_f32": [_vp, _i, _i, _i, _vp, _i, _vp, ctypes.c_float, _vp, _i, _vp, _vp],
    "trx_model_finalize": [_vp],
    "trx_model_sync": [_vp],
    "trx_model_generate": [_vp, _ip, _i, _i, _ip, _i],
    "trx_model_read": [_vp, _i, _vp, _sz],
    "trx_model_score": [_vp, _ip, _i, _vp, _vp],
    "trx_model_project_head": [_vp, _vp, _i, _vp],
    "trx_model_info": [_vp, _i, _i64p],
    "trx_model_tensor_ptr": [_vp, _i, _i, ctypes.POINTER(_vp), _i64p],
    "trx_model_packed_ptr": [_vp, _i, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp)],
    "trx_graph_begin": [_vp],
    "trx_graph_end": [_vp, ctypes.POINTER(_vp)],
    "trx_graph_launch": [_vp, _vp],
    "trx_graph_destroy": [_vp],
    "trx_probe_stream_read": [_vp, _sz, _vp, _i, _i, _vp],
    "trx_probe_empty": [_vp],
}
_RESTYPES = {"trx_last_error": ctypes.c_char_p}


class TrxError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{msg} (code {code})")
        self.code = code


_lib = None


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C trixium_amd/csrc` "
                               "(or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = L
    return _lib


def check(rc):
    if rc != TRX_OK:
        raise TrxError(rc, lib().trx_last_error().decode(errors="replace"))
    return rc


def call(name, *args):
    return check(getattr(lib(), name)(*args))


def device_count():
    n = ctypes.c_int(0)
    rc = lib().trx_device_count(ctypes.byref(n))
    return n.value if rc == TRX_OK else 0


def device_name():
    buf = ctypes.create_string_buffer(256)
    call("trx_device_name", buf, 256)
    return buf.value.decode()


class DeviceBuffer:
    """A device allocation (trx_malloc: 256 guard bytes past the end)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        call("trx_malloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a, stream=None):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a, stream)
        return b

    def upload(self, a, stream=None, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes, "upload past the end of the buffer"
        if a.nbytes:
            call("trx_memcpy_h2d", self.ptr + offset, a.ctypes.data, a.nbytes, stream)
            if stream is None:
                call("trx_stream_sync", None)

    def download(self, dtype, count=None, stream=None, offset=0):
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            call("trx_memcpy_d2h", out.ctypes.data, self.ptr + offset, out.nbytes, stream)
        return out

    def zero(self, stream=None):
        call("trx_memset_d8", self.ptr, 0, self.nbytes, stream)

    def free(self):
        if self.ptr:
            lib().trx_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize(stream=None):
    call("trx_stream_sync", stream)
