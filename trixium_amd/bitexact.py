"""GPU drop-in for the reference's engine matvec API (model/bitexact.py).

`matvec_ternary(scales_f16, codes, x8, B, R)` has the reference's signature and meaning
(model/bitexact.py:101-119): fp16 scales (M, K/128), codes (M, K) in {0,1,2}, x8 (K,) int8 ->
int32 (M,), asserting on int48 accumulator and int32 result overflow like the reference. The
matvec runs on the GPU through libtrixium_hip (trx_gemv_ternary_exact) on row packets encoded
from the arguments (trit5 by default). `group_sums` exposes the engine's exact per-group sums.
"""

import numpy as np

from . import layout as L
from .bons import encode_rows
from ._lib import DeviceBuffer, call, synchronize


def _packets(scales_f16, codes, kind):
    M, K = codes.shape
    assert K % 128 == 0 and scales_f16.shape == (M, K // 128)
    return encode_rows(kind, K, np.asarray(scales_f16, np.float16), np.asarray(codes, np.uint8))


def matvec_ternary_rows_gpu(rows_dev, kind, M, K, x8, B, R):
    """Exact matvec on resident row packets -> int32 (M,)."""
    xb = DeviceBuffer.from_array(np.asarray(x8, dtype=np.int8))
    yb = DeviceBuffer(4 * M)
    st = DeviceBuffer(4)
    st.zero()
    call("trx_gemv_ternary_exact", rows_dev.ptr, kind, M, K, xb.ptr, int(B), int(R), yb.ptr, st.ptr, None)
    synchronize()
    status = int(st.download(np.int32)[0])
    assert not (status & 1), "int48 accumulator overflow"
    assert not (status & 2), "int32 result overflow"
    return yb.download(np.int32, M)


def matvec_ternary(scales_f16, codes, x8, B, R, kind=L.KIND_TERNARY5):
    """The engine matvec (model/bitexact.py:101-119) on the GPU."""
    M, K = codes.shape
    rows = DeviceBuffer.from_array(_packets(scales_f16, codes, kind))
    return matvec_ternary_rows_gpu(rows, kind, M, K, x8, B, R)


def group_sums(scales_f16, codes, x8, kind=L.KIND_TERNARY5):
    """Exact per-group sums (M, K/128) of (code - 1) * x8 on the GPU."""
    M, K = codes.shape
    rows = DeviceBuffer.from_array(_packets(scales_f16, codes, kind))
    xb = DeviceBuffer.from_array(np.asarray(x8, dtype=np.int8))
    gs = DeviceBuffer(4 * M * (K // 128))
    call("trx_gemv_ternary_groupsums", rows.ptr, kind, M, K, xb.ptr, gs.ptr, None)
    synchronize()
    return gs.download(np.int32, M * (K // 128)).reshape(M, K // 128)


def matvec_float(scales_f16, codes, x, norm_w=None, eps=1e-6, kind=L.KIND_TERNARY5):
    """Float projection y = W x (fastref's matmul for one position) on the GPU, optionally with
    the fused RMSNorm of x."""
    M, K = codes.shape
    rows = DeviceBuffer.from_array(_packets(scales_f16, codes, kind))
    xb = DeviceBuffer.from_array(np.asarray(x, dtype=np.float32))
    nb = DeviceBuffer.from_array(np.asarray(norm_w, dtype=np.float32)) if norm_w is not None else None
    yb = DeviceBuffer(4 * M)
    call("trx_gemv_ternary_f32", rows.ptr, kind, M, K, xb.ptr, nb.ptr if nb else None, float(eps),
         yb.ptr, 0, None, None)
    synchronize()
    return yb.download(np.float32, M)


def pack_geometry(kind, M, K):
    """(packed bytes, workspace bytes) of the packed float GEMV for an M x K matrix."""
    import ctypes
    pb, wb = ctypes.c_size_t(), ctypes.c_size_t()
    call("trx_pack_geometry", int(kind), int(M), int(K), ctypes.byref(pb), ctypes.byref(wb))
    return pb.value, wb.value


class PackedMatrix:
    """A ternary matrix packed for the float GEMV (trx_pack_ternary) with its workspace."""

    def __init__(self, scales_f16, codes, kind=L.KIND_TERNARY5, swiglu=False):
        self.M, self.K = codes.shape
        self.kind = kind
        self.swiglu = bool(swiglu)
        rows = DeviceBuffer.from_array(_packets(scales_f16, codes, kind))
        pb, wb = pack_geometry(kind, self.M, self.K)
        self.packed = DeviceBuffer(pb)
        self.work = DeviceBuffer(wb)
        self.work.zero()
        call("trx_pack_ternary", rows.ptr, kind, self.M, self.K, int(self.swiglu), self.packed.ptr, None)
        synchronize()

    def matvec(self, x, norm_w=None, eps=1e-6, epilogue=0, resid=None):
        """y = W xhat with the epilogue (TRX_EPI_*); SwiGLU returns M/2 values."""
        xb = DeviceBuffer.from_array(np.asarray(x, dtype=np.float32))
        nb = DeviceBuffer.from_array(np.asarray(norm_w, dtype=np.float32)) if norm_w is not None else None
        n_out = self.M // 2 if epilogue == 2 else self.M
        if resid is not None:
            yb = DeviceBuffer.from_array(np.asarray(resid, dtype=np.float32))
        else:
            yb = DeviceBuffer(4 * n_out)
        call("trx_gemv_packed_f32", self.packed.ptr, self.kind, self.M, self.K, xb.ptr,
             nb.ptr if nb else None, float(eps), yb.ptr, int(epilogue), yb.ptr if resid is not None else None,
             self.work.ptr, None)
        synchronize()
        return yb.download(np.float32, n_out)
