"""GPU drop-in for the reference's engine matvec API (model/bitexact.py).

`matvec_ternary(scales_f16, codes, x8, B, R)` has the reference's signature and meaning
(model/bitexact.py:101-119): fp16 scales (M, K/128), codes (M, K) in {0,1,2}, x8 (K,) int8 ->
int32 (M,), asserting on int48 accumulator and int32 result overflow like the reference. The
matvec runs on the GPU through libtrixium_hip (trx_gemv_ternary_exact) on row packets encoded
from the arguments (trit5 by default). `group_sums` exposes the engine's exact per-group sums.
"""

import ctypes

import numpy as np

from . import layout as L
from .bons import encode_rows
from ._lib import DeviceBuffer, PartialSums, call, synchronize


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


ROWS_STAGED_BYTES = 114688   # n * K bound of one trx_gemv_ternary_exact_rows call


def matvec_ternary_rows_multi_gpu(rows_dev, kind, M, K, x8_rows, B, R):
    """Multi-row exact matvec on resident row packets: x8_rows (n, K) int8, n in 1..8 -> int32
    (n, M), one weight pass (trx_gemv_ternary_exact_rows)."""
    x = np.ascontiguousarray(x8_rows, dtype=np.int8)
    assert x.ndim == 2 and x.shape[1] == K
    n = x.shape[0]
    xb = DeviceBuffer.from_array(x)
    yb = DeviceBuffer(4 * n * M)
    st = DeviceBuffer(4)
    st.zero()
    call("trx_gemv_ternary_exact_rows", rows_dev.ptr, kind, M, K, xb.ptr, n, int(B), int(R), yb.ptr,
         st.ptr, None)
    synchronize()
    status = int(st.download(np.int32)[0])
    assert not (status & 1), "int48 accumulator overflow"
    assert not (status & 2), "int32 result overflow"
    return yb.download(np.int32, n * M).reshape(n, M)


def matvec_ternary_rows(scales_f16, codes, x8_rows, B, R, kind=L.KIND_TERNARY5):
    """The engine's multi-row matvec (model/bitexact.py:121-125) on the GPU: x8_rows (n, K) int8
    -> int32 (n, M), each row the single-row matvec of its x. One pass takes at most 8 rows and
    ROWS_STAGED_BYTES of x; more run in several passes."""
    M, K = codes.shape
    rows = DeviceBuffer.from_array(_packets(scales_f16, codes, kind))
    x = np.asarray(x8_rows, dtype=np.int8)
    step = max(1, min(8, ROWS_STAGED_BYTES // K))
    return np.concatenate([matvec_ternary_rows_multi_gpu(rows, kind, M, K, x[i:i + step], B, R)
                           for i in range(0, x.shape[0], step)])


def quantize_f_pow2(x):
    """The firmware's activation quantizer on the GPU (model/mirror.py:45-51): (int8 [K], e8)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))
    xb = DeviceBuffer.from_array(x)
    qb = DeviceBuffer(max(16, x.size))
    eb = DeviceBuffer(4)
    call("trx_quantize_f_pow2", xb.ptr, int(x.size), qb.ptr, eb.ptr, None)
    synchronize()
    return qb.download(np.int8, x.size), int(eb.download(np.int32)[0])


def matvec_quantized(scales_f16, codes, x, B, R, kind=L.KIND_TERNARY5):
    """The projection as the firmware runs it through the engine (model/mirror.py:663-678): x
    quantized to int8 with a power-of-two exponent, the exact matvec, the int32 result scaled by
    2^(e8 + R - B). float32 (M,). Asserts as matvec_ternary on overflow."""
    M, K = codes.shape
    rows = DeviceBuffer.from_array(_packets(scales_f16, codes, kind))
    xb = DeviceBuffer.from_array(np.asarray(x, dtype=np.float32))
    wb = ctypes.c_size_t()
    call("trx_gemv_quantized_geometry", M, K, ctypes.byref(wb))
    work = DeviceBuffer(wb.value)
    yb = DeviceBuffer(4 * M)
    st = DeviceBuffer(4)
    st.zero()
    call("trx_gemv_ternary_quantized", rows.ptr, kind, M, K, xb.ptr, int(B), int(R), yb.ptr, work.ptr, st.ptr, None)
    synchronize()
    status = int(st.download(np.int32)[0])
    assert not (status & 1), "int48 accumulator overflow"
    assert not (status & 2), "int32 result overflow"
    return yb.download(np.float32, M)


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
    pb, wb = ctypes.c_size_t(), ctypes.c_size_t()
    call("trx_pack_geometry", int(kind), int(M), int(K), ctypes.byref(pb), ctypes.byref(wb))
    return pb.value, wb.value


def batched_matvec(mats, xs, kind=L.KIND_TERNARY5, n_mat=None):
    """y_i = W_(i % len(mats)) x_i for i < n_mat (default len(mats)) in one dispatch
    (trx_gemv_packed_batched_f32): the packed copies back to back at a 256-byte multiple stride.
    xs: (n_mat, K), or one (K,) vector for every matrix (x_stride 0). Returns float32 (n_mat, M)."""
    n = len(mats)
    n_mat = n if n_mat is None else int(n_mat)
    M, K = mats[0][1].shape
    shared = np.ndim(xs) == 1
    pb, _ = pack_geometry(kind, M, K)
    stride = -(-pb // 256) * 256
    packed = DeviceBuffer(stride * n)
    for i, (sc, cd) in enumerate(mats):
        assert cd.shape == (M, K)
        rows = DeviceBuffer.from_array(_packets(sc, cd, kind))
        call("trx_pack_ternary", rows.ptr, kind, M, K, 0, packed.ptr + i * stride, None)
        synchronize()
    wb = ctypes.c_size_t()
    call("trx_pack_batched_geometry", kind, M, K, n_mat, ctypes.byref(wb))
    work = DeviceBuffer(wb.value)
    xb = DeviceBuffer.from_array(np.ascontiguousarray(np.asarray(xs, dtype=np.float32).reshape(-1 if shared else n_mat, K)))
    yb = DeviceBuffer(4 * n_mat * M)
    call("trx_gemv_packed_batched_f32", packed.ptr, stride, n_mat, n, kind, M, K, xb.ptr, 0 if shared else K, yb.ptr, M,
         work.ptr, None)
    synchronize()
    return yb.download(np.float32, n_mat * M).reshape(n_mat, M)


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

    def partials_geometry(self):
        """(S, rows_p, bps) of trx_pack_partials_geometry."""
        S, rp, bps = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        call("trx_pack_partials_geometry", self.kind, self.M, self.K, ctypes.byref(S), ctypes.byref(rp), ctypes.byref(bps))
        return S.value, rp.value, bps.value

    def partials(self, x, norm_w=None, eps=1e-6):
        """The split-K partial sums only (trx_gemv_packed_parts_f32 with `out`): a dict with the
        device buffers part ([S][rows_p]) and ss (the slice sums of x^2 with an RMSNorm), S,
        rows_p and K, for a consumer's matvec_from."""
        S, rp, bps = self.partials_geometry()
        xb = DeviceBuffer.from_array(np.asarray(x, dtype=np.float32))
        nb = DeviceBuffer.from_array(np.asarray(norm_w, dtype=np.float32)) if norm_w is not None else None
        part, ss = DeviceBuffer(4 * S * rp), DeviceBuffer(4 * bps * S)
        ps = PartialSums(out=part.ptr, out_ss=ss.ptr if nb else None)
        call("trx_gemv_packed_parts_f32", self.packed.ptr, self.kind, self.M, self.K, xb.ptr, nb.ptr if nb else None,
             float(eps), None, 2 if self.swiglu else 0, None, self.work.ptr, ctypes.byref(ps), None)
        synchronize()
        return {"part": part, "ss": ss if nb else None, "S": S, "rows_p": rp, "K": self.K, "swiglu": self.swiglu}

    def matvec_from(self, src, resid_x=None, norm_w=None, eps=1e-6, epilogue=0, resid=None):
        """y = W xhat with x from a producer's partial sums (`src` from partials): SwiGLU of a
        gate|up producer's sums, or resid_x plus a residual producer's sums. Returns (y, x)."""
        ps = PartialSums(in_=src["part"].ptr, S=src["S"], rows_p=src["rows_p"])
        if src["swiglu"]:
            ps.F = self.K
            if src["ss"] is not None:
                ps.in_ss = src["ss"].ptr
                ps.in_K = src["K"]
        else:
            rb = DeviceBuffer.from_array(np.asarray(resid_x, dtype=np.float32))
            ps.resid = rb.ptr
        act = DeviceBuffer(4 * self.K)
        ps.act = act.ptr
        nb = DeviceBuffer.from_array(np.asarray(norm_w, dtype=np.float32)) if norm_w is not None else None
        yb = DeviceBuffer.from_array(np.asarray(resid, dtype=np.float32)) if resid is not None else DeviceBuffer(4 * self.M)
        call("trx_gemv_packed_parts_f32", self.packed.ptr, self.kind, self.M, self.K, None, nb.ptr if nb else None,
             float(eps), yb.ptr, int(epilogue), yb.ptr if resid is not None else None, self.work.ptr,
             ctypes.byref(ps), None)
        synchronize()
        return yb.download(np.float32, self.M), act.download(np.float32, self.K)
