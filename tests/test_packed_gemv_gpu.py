"""Packed float GEMV (table lookup over the slice-major copy) on the GPU against float64
evaluations of the same product: plain, RMSNorm prologue, residual and SwiGLU epilogues, odd
group counts and ragged row counts, both code formats, determinism and workspace reuse."""

import numpy as np
import pytest

from trixium_amd import layout as L

pytestmark = pytest.mark.gpu

KINDS = [L.KIND_TERNARY5, L.KIND_TERNARY]
EPI_STORE, EPI_RESID, EPI_SWIGLU = 0, 1, 2
# fp32 table entries and sums against float64: error relative to sum |w| |x| per row.
TOL = 2e-6


def _rand(M, K, seed, p0=0.4, max_code=2):
    r = np.random.default_rng(seed)
    u = r.random((M, K))
    codes = np.where(u < (1 - p0) / 2, 0, np.where(u < (1 + p0) / 2, 1, 2)).astype(np.uint8)
    if max_code == 3:
        codes[r.random((M, K)) < 0.1] = 3
    scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
    return codes, scales


def _w64(codes, scales):
    M, K = codes.shape
    W = (codes.astype(np.float64) - 1).reshape(M, -1, 128) * scales.astype(np.float64)[:, :, None]
    return W.reshape(M, K)


@pytest.fixture(scope="module")
def gpu():
    from trixium_amd import _lib
    if _lib.device_count() < 1:
        pytest.fail("no GPU visible to libtrixium_hip")
    from trixium_amd import bitexact
    return bitexact


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,K", [(1, 128), (3, 256), (7, 384), (33, 768), (257, 2048), (1000, 4096),
                                 (4099, 256), (50, 12288), (130, 4224)])
def test_packed_matvec_vs_float64(gpu, kind, M, K):
    print(f"packed matvec kind={kind} M={M} K={K}", flush=True)
    codes, scales = _rand(M, K, K * 7 + M)
    x = np.random.default_rng(M + 1).normal(0, 1, K).astype(np.float32)
    pm = gpu.PackedMatrix(scales, codes, kind)
    y = pm.matvec(x)
    W = _w64(codes, scales)
    ref = W @ x.astype(np.float64)
    mag = np.abs(W) @ np.abs(x.astype(np.float64))
    assert np.max(np.abs(y - ref) / mag) < TOL


def test_packed_matvec_code3_two_bit(gpu):
    """2-bit code 3 decodes to weight 2 (code - 1), as the reference's decode does."""
    M, K = 64, 1024
    codes, scales = _rand(M, K, 3, max_code=3)
    x = np.random.default_rng(4).normal(0, 1, K).astype(np.float32)
    y = gpu.PackedMatrix(scales, codes, L.KIND_TERNARY).matvec(x)
    W = _w64(codes, scales)
    assert np.max(np.abs(y - W @ x) / (np.abs(W) @ np.abs(x))) < TOL


@pytest.mark.parametrize("kind", KINDS)
def test_packed_matvec_zero_weights_and_zero_x(gpu, kind):
    M, K = 40, 512
    codes = np.ones((M, K), np.uint8)
    scales = np.full((M, K // 128), 0.03, np.float16)
    x = np.random.default_rng(0).normal(0, 1, K).astype(np.float32)
    assert np.all(gpu.PackedMatrix(scales, codes, kind).matvec(x) == 0)
    codes, scales = _rand(M, K, 1)
    assert np.all(gpu.PackedMatrix(scales, codes, kind).matvec(np.zeros(K, np.float32)) == 0)


@pytest.mark.parametrize("kind", KINDS)
def test_packed_matvec_rmsnorm_prologue(gpu, kind):
    M, K = 300, 2048
    codes, scales = _rand(M, K, 5)
    r = np.random.default_rng(6)
    x = r.normal(0, 3, K).astype(np.float32)
    w = r.uniform(0.8, 1.2, K).astype(np.float32)
    y = gpu.PackedMatrix(scales, codes, kind).matvec(x, norm_w=w, eps=1e-6)
    xn = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    W = _w64(codes, scales)
    assert np.max(np.abs(y - W @ xn) / (np.abs(W) @ np.abs(xn))) < 1e-5


@pytest.mark.parametrize("kind", KINDS)
def test_packed_matvec_residual(gpu, kind):
    M, K = 515, 1024
    codes, scales = _rand(M, K, 7)
    r = np.random.default_rng(8)
    x = r.normal(0, 1, K).astype(np.float32)
    res = r.normal(0, 2, M).astype(np.float32)
    y = gpu.PackedMatrix(scales, codes, kind).matvec(x, epilogue=EPI_RESID, resid=res)
    W = _w64(codes, scales)
    ref = res.astype(np.float64) + W @ x
    assert np.max(np.abs(y - ref) / (np.abs(W) @ np.abs(x) + np.abs(res))) < TOL


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("F,K", [(2, 256), (6, 384), (300, 1024), (1536, 4096)])
def test_packed_matvec_swiglu(gpu, kind, F, K):
    codes, scales = _rand(2 * F, K, F + K)
    x = np.random.default_rng(F).normal(0, 1, K).astype(np.float32)
    y = gpu.PackedMatrix(scales, codes, kind, swiglu=True).matvec(x, epilogue=EPI_SWIGLU)
    W = _w64(codes, scales)
    g, u = W[:F] @ x, W[F:] @ x
    ref = g / (1 + np.exp(-g)) * u
    mg, mu = np.abs(W[:F]) @ np.abs(x), np.abs(W[F:]) @ np.abs(x)
    err = np.abs(y - ref) / (mg * (np.abs(u) + mu) + 1e-30)
    assert y.shape == (F,) and np.max(err) < 1e-5


def test_packed_matvec_deterministic_and_reusable(gpu):
    """Bitwise identical repeats; the workspace counters are left ready after every call."""
    codes, scales = _rand(6144, 4096, 9)
    pm = gpu.PackedMatrix(scales, codes)
    r = np.random.default_rng(1)
    xs = [r.normal(0, 1, 4096).astype(np.float32) for _ in range(3)]
    first = [pm.matvec(x) for x in xs]
    again = [pm.matvec(x) for x in xs]
    W = _w64(codes, scales)
    for x, a, b in zip(xs, first, again):
        assert np.array_equal(a, b)
        assert np.max(np.abs(a - W @ x) / (np.abs(W) @ np.abs(x))) < TOL


def test_packed_matvec_agrees_with_int16_path(gpu):
    """The packed path (fp32 x) and the row-packet path (x quantised to int16 per group)."""
    codes, scales = _rand(512, 4096, 11)
    x = np.random.default_rng(2).normal(0, 1, 4096).astype(np.float32)
    a = gpu.PackedMatrix(scales, codes).matvec(x)
    b = gpu.matvec_float(scales, codes, x)
    W = _w64(codes, scales)
    assert np.max(np.abs(a - b) / (np.abs(W) @ np.abs(x))) < 2e-4


def test_packed_matrices_share_a_workspace(gpu):
    """Matrices of different row-tile counts interleaved on one workspace (as the decoder's
    projections share one): every result matches float64."""
    from trixium_amd import _lib
    shapes = [(300, 512), (5000, 512), (40, 1024), (9000, 256)]
    mats, refs = [], []
    for i, (M, K) in enumerate(shapes):
        codes, scales = _rand(M, K, 40 + i)
        mats.append(gpu.PackedMatrix(scales, codes))
        refs.append(_w64(codes, scales))
    work = _lib.DeviceBuffer(max(m.work.nbytes for m in mats))
    work.zero()
    for m in mats:
        m.work = work
    r = np.random.default_rng(5)
    for rep in range(3):
        for m, W in zip(mats, refs):
            x = r.normal(0, 1, m.K).astype(np.float32)
            y = m.matvec(x)
            assert np.max(np.abs(y - W @ x) / (np.abs(W) @ np.abs(x))) < TOL, (rep, m.M, m.K)


def _silu(v):
    return v / (1 + np.exp(-v))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("E,F", [(256, 256), (1024, 768), (2048, 6144), (5120, 4352), (384, 640)])
def test_partial_sums_gate_up_to_down(gpu, kind, E, F):
    """gate|up (RMSNorm) stores its partial sums; down takes them: SwiGLU with the RMSNorm scale
    applied to g and u, then the residual epilogue. y, and the activation down stores, against
    float64."""
    print(f"gate|up -> down kind={kind} E={E} F={F}", flush=True)
    cg, sg = _rand(2 * F, E, E + F)
    cd, sd = _rand(E, F, F + 3)
    r = np.random.default_rng(E)
    x = r.normal(0, 2, E).astype(np.float32)
    w = r.uniform(0.8, 1.2, E).astype(np.float32)
    res = r.normal(0, 1, E).astype(np.float32)
    gu = gpu.PackedMatrix(sg, cg, kind, swiglu=True)
    dn = gpu.PackedMatrix(sd, cd, kind)
    src = gu.partials(x, norm_w=w, eps=1e-6)
    y, h = dn.matvec_from(src, epilogue=EPI_RESID, resid=res)
    xn = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    Wg = _w64(cg, sg)
    g, u = Wg[:F] @ xn, Wg[F:] @ xn
    h64 = _silu(g) * u
    hmag = (np.abs(Wg[:F]) @ np.abs(xn)) * (np.abs(u) + np.abs(Wg[F:]) @ np.abs(xn))
    assert np.max(np.abs(h - h64) / (hmag + 1e-30)) < 1e-5
    Wd = _w64(cd, sd)
    ref = res + Wd @ h64
    assert np.max(np.abs(y - ref) / (np.abs(Wd) @ np.abs(h64) + np.abs(res))) < 1e-5


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("E,K", [(256, 256), (2048, 2048), (4096, 6144), (1152, 640)])
def test_partial_sums_residual_to_normed_gemv(gpu, kind, E, K):
    """A residual producer (o: E x K) stores its partial sums; the next GEMV (E -> 3E/2 rows, with
    an RMSNorm) takes x = resid + their sums and stores that x. Both against float64."""
    print(f"residual -> normed kind={kind} E={E} K={K}", flush=True)
    co, so = _rand(E, K, E * 3 + K)
    M2 = 3 * E // 2
    c2, s2 = _rand(M2, E, E + 11)
    r = np.random.default_rng(K)
    xo = r.normal(0, 1, K).astype(np.float32)
    resid = r.normal(0, 3, E).astype(np.float32)
    w = r.uniform(0.8, 1.2, E).astype(np.float32)
    o = gpu.PackedMatrix(so, co, kind)
    m2 = gpu.PackedMatrix(s2, c2, kind)
    y, xnew = m2.matvec_from(o.partials(xo), resid_x=resid, norm_w=w, eps=1e-6)
    Wo = _w64(co, so)
    x64 = resid.astype(np.float64) + Wo @ xo
    assert np.max(np.abs(xnew - x64) / (np.abs(Wo) @ np.abs(xo) + np.abs(resid))) < 2e-6
    xn = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6) * w
    W2 = _w64(c2, s2)
    assert np.max(np.abs(y - W2 @ xn) / (np.abs(W2) @ np.abs(xn))) < 1e-5


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,K,n", [(2048, 2048, 5), (257, 640, 3), (6144, 2048, 2), (2048, 6144, 2), (1, 128, 4)])
def test_batched_matvec_equals_single_launches(gpu, kind, M, K, n):
    """Many independent GEMVs in one dispatch (trx_gemv_packed_batched_f32): every y_i within
    the float64 tolerance and bitwise equal to the single-matrix packed GEMV of the same W_i, x_i
    (the same per-slice partial sums, added in slice order)."""
    print(f"batched matvec kind={kind} M={M} K={K} n={n}", flush=True)
    mats = [_rand(M, K, 1000 * i + K + M)[::-1] for i in range(n)]
    xs = np.random.default_rng(K + n).normal(0, 1, (n, K)).astype(np.float32)
    y = gpu.batched_matvec(mats, xs, kind)
    for i, (sc, cd) in enumerate(mats):
        W = _w64(cd, sc)
        ref = W @ xs[i].astype(np.float64)
        mag = np.abs(W) @ np.abs(xs[i].astype(np.float64))
        assert np.max(np.abs(y[i] - ref) / np.maximum(mag, 1e-30)) < TOL
        single = gpu.PackedMatrix(sc, cd, kind).matvec(xs[i])
        assert np.array_equal(y[i], single), i


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,K,n_mat,copies", [(257, 2048, 300, 5), (2048, 2048, 96, 3), (128, 256, 2, 2),
                                              (300, 640, 7, 3), (640, 640, 1, 1)])
def test_batched_matvec_with_one_x(gpu, kind, M, K, n_mat, copies):
    """One x for every matrix (x_stride 0): a block builds the tables of two K-slices once and
    streams them over several matrices, cycling over the copies (K = 256 and 640: an odd slice
    count, the last block's second slice missing). Every y_i within the float64 tolerance, equal
    bit for bit to every other y_j of its copy, and within the tolerance of the single-matrix
    packed GEMV (whose partial sums are added one slice at a time, not in pairs)."""
    print(f"batched matvec, one x: kind={kind} M={M} K={K} n_mat={n_mat} copies={copies}", flush=True)
    mats = [_rand(M, K, 77 * i + K + M)[::-1] for i in range(copies)]
    x = np.random.default_rng(K + n_mat).normal(0, 1, K).astype(np.float32)
    y = gpu.batched_matvec(mats, x, kind, n_mat=n_mat)
    for c, (sc, cd) in enumerate(mats):
        W = _w64(cd, sc)
        ref = W @ x.astype(np.float64)
        mag = np.maximum(np.abs(W) @ np.abs(x.astype(np.float64)), 1e-30)
        single = gpu.PackedMatrix(sc, cd, kind).matvec(x)
        assert np.max(np.abs(single - ref) / mag) < TOL
        for i in range(c, n_mat, copies):
            assert np.max(np.abs(y[i] - ref) / mag) < TOL, i
            assert np.max(np.abs(y[i] - single) / mag) < TOL, i
            assert np.array_equal(y[i], y[c]), i
