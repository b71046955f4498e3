"""trx_gemv_packed_f32_noalloc (the packed GEMV with its workspace in the library's fixed device
array) against trx_gemv_packed_f32 with a caller workspace, through the C ABI: two calls in a
row, the second with a smaller matrix, plus an RMSNorm + residual call and a SwiGLU call; every
result bitwise equal (same kernel, same geometry). A matrix whose workspace exceeds the array
is refused."""

import ctypes

import numpy as np
import pytest

from trixium_amd import _lib, layout as L
from trixium_amd.bitexact import PackedMatrix

pytestmark = pytest.mark.gpu


def _rand(M, K, seed):
    r = np.random.default_rng(seed)
    u = r.random((M, K))
    codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
    return r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16), codes


def _noalloc(pm, x, norm_w=None, epilogue=0, resid=None):
    n_out = pm.M // 2 if epilogue == 2 else pm.M
    xb = _lib.DeviceBuffer.from_array(np.asarray(x, np.float32))
    nb = _lib.DeviceBuffer.from_array(np.asarray(norm_w, np.float32)) if norm_w is not None else None
    yb = _lib.DeviceBuffer.from_array(np.asarray(resid, np.float32)) if resid is not None else _lib.DeviceBuffer(4 * n_out)
    _lib.call("trx_gemv_packed_f32_noalloc", pm.packed.ptr, pm.kind, pm.M, pm.K, xb.ptr, nb.ptr if nb else None,
              ctypes.c_float(1e-6), yb.ptr, int(epilogue), yb.ptr if resid is not None else None, None)
    _lib.synchronize()
    return yb.download(np.float32, n_out)


@pytest.mark.parametrize("kind", [L.KIND_TERNARY5, L.KIND_TERNARY])
def test_noalloc_gemv_equals_workspace_gemv(kind):
    print(f"no-alloc GEMV kind={kind}", flush=True)
    big = PackedMatrix(*_rand(6144, 4096, 1), kind)
    small = PackedMatrix(*_rand(300, 640, 2), kind)
    rng = np.random.default_rng(3)
    xb, xs = rng.standard_normal(4096).astype(np.float32), rng.standard_normal(640).astype(np.float32)
    a1, a2 = _noalloc(big, xb), _noalloc(small, xs)
    assert np.array_equal(a1, big.matvec(xb))
    assert np.array_equal(a2, small.matvec(xs))
    g = rng.uniform(0.8, 1.2, 4096).astype(np.float32)
    res = rng.standard_normal(6144).astype(np.float32)
    assert np.array_equal(_noalloc(big, xb, g, 1, res), big.matvec(xb, g, epilogue=1, resid=res))
    swi = PackedMatrix(*_rand(2048, 1024, 4), kind, swiglu=True)
    x3 = rng.standard_normal(1024).astype(np.float32)
    assert np.array_equal(_noalloc(swi, x3, epilogue=2), swi.matvec(x3, epilogue=2))
    # The same big call again after the small ones (the array keeps the last call's contents).
    assert np.array_equal(_noalloc(big, xb), a1)


def test_noalloc_gemv_refuses_an_oversized_workspace():
    """A 151936 x 12288 matrix needs ~29 MB of partial sums: more than the fixed array."""
    from trixium_amd.bitexact import pack_geometry
    _, wb = pack_geometry(L.KIND_TERNARY5, 151936, 12288)
    assert wb > 24 << 20
    x = _lib.DeviceBuffer(4 * 12288)
    y = _lib.DeviceBuffer(4 * 151936)
    with pytest.raises(_lib.TrxError):
        _lib.call("trx_gemv_packed_f32_noalloc", x.ptr, L.KIND_TERNARY5, 151936, 12288, x.ptr, None,
                  ctypes.c_float(1e-6), y.ptr, 0, None, None)


_CAPTURE_SCRIPT = r"""
import ctypes, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from trixium_amd import _lib, layout as L
from trixium_amd.bitexact import PackedMatrix
r = np.random.default_rng(5)
u = r.random((1024, 2048))
codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
pm = PackedMatrix(r.uniform(0.01, 0.05, (1024, 16)).astype(np.float16), codes, L.KIND_TERNARY5)
x = r.standard_normal(2048).astype(np.float32)
want = pm.matvec(x)
s = ctypes.c_void_p()
_lib.call("trx_stream_create", ctypes.byref(s))
xb = _lib.DeviceBuffer.from_array(x)
yb = _lib.DeviceBuffer(4 * 1024)
exe = ctypes.c_void_p()
# The process's first no-alloc call, inside the capture: the array's address lookup happens then
# and its counter clearing is recorded into the graph.
_lib.call("trx_graph_begin", s)
_lib.call("trx_gemv_packed_f32_noalloc", pm.packed.ptr, pm.kind, 1024, 2048, xb.ptr, None, ctypes.c_float(1e-6),
          yb.ptr, 0, None, s)
_lib.call("trx_graph_end", s, ctypes.byref(exe))
ok = True
for rep in range(3):
    yb.zero(s)
    _lib.call("trx_graph_launch", exe, s)
    _lib.call("trx_stream_sync", s)
    ok = ok and np.array_equal(yb.download(np.float32, 1024), want)
_lib.call("trx_graph_destroy", exe)
_lib.call("trx_stream_destroy", s)
print("replays equal:", ok, flush=True)
sys.exit(0 if ok else 1)
"""


def test_noalloc_gemv_first_call_under_graph_capture():
    """The no-alloc GEMV's first call in a process made while a stream is being captured (as a
    caller under hipGraph capture makes it): the graph replays three times, each equal to the
    GEMV with a caller workspace."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("no-alloc GEMV: first call under capture, in a fresh process", flush=True)
    p = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, root], capture_output=True, text=True, timeout=120)
    print(p.stdout, p.stderr[-2000:], flush=True)
    assert p.returncode == 0
