"""Ternary GEMV on the GPU against the oracle: exact group sums and engine results bit-exact,
the float path within tolerance of a float64 evaluation, on both code formats."""

import hashlib

import numpy as np
import pytest

from oracle import bitexact as ob
from trixium_amd import layout as L, configs as C

pytestmark = pytest.mark.gpu

KINDS = [L.KIND_TERNARY5, L.KIND_TERNARY]


def _rand(M, K, seed, p0=0.4):
    r = np.random.default_rng(seed)
    u = r.random((M, K))
    codes = np.where(u < (1 - p0) / 2, 0, np.where(u < (1 + p0) / 2, 1, 2)).astype(np.uint8)
    scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
    x8 = r.integers(-127, 128, K, dtype=np.int8)
    return codes, scales, x8


@pytest.fixture(scope="module")
def gpu():
    from trixium_amd import _lib
    if _lib.device_count() < 1:
        pytest.fail("no GPU visible to libtrixium_hip")
    print("device:", _lib.device_name(), flush=True)
    from trixium_amd import bitexact
    return bitexact


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,K", [(1, 128), (7, 256), (33, 768), (64, 2048), (100, 4096), (17, 6144),
                                 (9, 12288), (5, 17408), (3, 5120)])
def test_group_sums_bit_exact(gpu, kind, M, K):
    print(f"group sums kind={kind} M={M} K={K}", flush=True)
    codes, scales, x8 = _rand(M, K, M * 131 + K)
    got = gpu.group_sums(scales, codes, x8, kind=kind)
    assert np.array_equal(got, ob.group_sums(codes, x8))


@pytest.mark.parametrize("kind", KINDS)
def test_group_sums_extremes(gpu, kind):
    """All +1 codes against x8 = 127 (the |gs| = 16256 bound), all -1 against -127, zeros."""
    K = 1024
    for code, xv in ((2, 127), (0, -127), (2, -128), (1, 55)):
        codes = np.full((3, K), code, np.uint8)
        scales = np.full((3, K // 128), 0.02, np.float16)
        x8 = np.full(K, xv, np.int8)
        assert np.array_equal(gpu.group_sums(scales, codes, x8, kind=kind), ob.group_sums(codes, x8))


@pytest.mark.parametrize("kind", KINDS)
def test_matvec_exact_microbench_fixtures(gpu, golden, kind):
    """The four microbench shapes, against the sha256 the reference's matvec_ternary produced."""
    for (M, K) in C.MICROBENCH_SHAPES:
        r = np.random.default_rng(M * 7919 + K)
        u = r.random((M, K))
        codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
        scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
        x8 = r.integers(-127, 128, K, dtype=np.int8)
        g = golden[f"matvec/{M}x{K}"]
        print(f"exact matvec kind={kind} {M}x{K}", flush=True)
        res = gpu.matvec_ternary(scales, codes, x8, g["B"], g["R"], kind=kind)
        assert hashlib.sha256(res.astype("<i4").tobytes()).hexdigest() == g["sha256"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,K,n", [(1, 128, 1), (3, 640, 8), (33, 768, 3), (100, 4096, 8),
                                   (17, 6144, 5), (9, 12288, 8), (5, 17408, 8), (70, 2048, 2)])
def test_matvec_rows_vs_oracle(gpu, kind, M, K, n):
    """One weight pass against n x8 rows: every row bit-exact with the oracle's single-row matvec
    (wide-exponent scales, so both shift directions occur) and with the single-row GPU call."""
    r = np.random.default_rng(M * 31 + K + n)
    codes = r.integers(0, 3, (M, K), dtype=np.uint8)
    scales = (np.exp2(r.uniform(-20, 3, (M, K // 128))) * r.choice([-1, 1], (M, K // 128))).astype(np.float16)
    xs = r.integers(-128, 128, (n, K), dtype=np.int8)
    xs[0, : K // 2] = 127
    _, e16 = ob.fp16_decompose(scales)
    B = ob.choose_scale_bias(e16)
    R = ob.choose_result_shift(scales, B)
    print(f"multi-row matvec kind={kind} {M}x{K} n={n}", flush=True)
    got = gpu.matvec_ternary_rows(scales, codes, xs, B, R, kind=kind)
    assert got.shape == (n, M)
    assert np.array_equal(got, ob.matvec_ternary_rows(scales, codes, xs, B, R))
    assert np.array_equal(got[-1], gpu.matvec_ternary(scales, codes, xs[-1], B, R, kind=kind))


@pytest.mark.parametrize("kind", KINDS)
def test_matvec_rows_microbench_fixtures(gpu, golden, kind):
    """The microbench shapes in a 7-row pass (11 rows: passes of 8 and 3): the fixture's x at rows
    0 and 9 matches the sha256 the reference's matvec_ternary produced. Every group shift is a
    left shift at these scales, so the negated x gives the negated accumulator and results that
    differ from the negated ones by the final floor shift alone (at most 1)."""
    for (M, K) in C.MICROBENCH_SHAPES:
        r = np.random.default_rng(M * 7919 + K)
        u = r.random((M, K))
        codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
        scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
        x8 = r.integers(-127, 128, K, dtype=np.int8)
        g = golden[f"matvec/{M}x{K}"]
        xs = np.random.default_rng(K).integers(-127, 128, (11, K), dtype=np.int8)
        xs[0] = x8
        xs[9] = x8
        xs[4] = -x8
        print(f"multi-row microbench kind={kind} {M}x{K}", flush=True)
        res = gpu.matvec_ternary_rows(scales, codes, xs, g["B"], g["R"], kind=kind)
        for i in (0, 9):
            assert hashlib.sha256(res[i].astype("<i4").tobytes()).hexdigest() == g["sha256"]
        assert np.all(np.abs(res[4].astype(np.int64) + res[0]) <= 1)


def test_matvec_rows_overflow_asserts(gpu):
    """An overflowing row among good ones trips the reference's int32 result assertion."""
    codes = np.full((2, 12288), 2, np.uint8)
    scales = np.full((2, 96), 0.5, np.float16)
    xs = np.zeros((3, 12288), np.int8)
    xs[1] = 127
    _, e16 = ob.fp16_decompose(scales)
    B = ob.choose_scale_bias(e16)
    with pytest.raises(AssertionError, match="int32 result overflow"):
        gpu.matvec_ternary_rows(scales, codes, xs, B, 0)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,K", [(5, 256), (129, 4096), (31, 12288)])
def test_matvec_exact_wide_scales(gpu, kind, M, K):
    """Scales over a wide exponent range (negative and positive per-group shifts)."""
    r = np.random.default_rng(K + M)
    codes = r.integers(0, 3, (M, K), dtype=np.uint8)
    scales = (np.exp2(r.uniform(-20, 3, (M, K // 128))) * r.choice([-1, 1], (M, K // 128))).astype(np.float16)
    x8 = r.integers(-127, 128, K, dtype=np.int8)
    _, e16 = ob.fp16_decompose(scales)
    B = ob.choose_scale_bias(e16)
    R = ob.choose_result_shift(scales, B)
    assert np.array_equal(gpu.matvec_ternary(scales, codes, x8, B, R, kind=kind),
                          ob.matvec_ternary(scales, codes, x8, B, R))


def test_matvec_exact_overflow_asserts(gpu):
    """A result shift too small for the int32 result trips the same assertion as the reference."""
    codes = np.full((2, 12288), 2, np.uint8)
    scales = np.full((2, 96), 0.5, np.float16)
    x8 = np.full(12288, 127, np.int8)
    _, e16 = ob.fp16_decompose(scales)
    B = ob.choose_scale_bias(e16)
    with pytest.raises(AssertionError, match="int32 result overflow"):
        gpu.matvec_ternary(scales, codes, x8, B, 0)
    with pytest.raises(AssertionError):
        ob.matvec_ternary(scales, codes, x8, B, 0)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,K", [(3, 256), (257, 2048), (1000, 4096), (50, 12288)])
def test_matvec_float_vs_float64(gpu, kind, M, K):
    """fp32 x quantised to int16 per group inside the kernel: relative error < 2e-4 of the
    row's magnitude scale against the exact float64 product."""
    codes, scales, _ = _rand(M, K, K * 3 + M)
    x = np.random.default_rng(M).normal(0, 1, K).astype(np.float32)
    y = gpu.matvec_float(scales, codes, x, kind=kind)
    W = (codes.astype(np.float64) - 1).reshape(M, -1, 128) * scales.astype(np.float64)[:, :, None]
    ref = W.reshape(M, K) @ x.astype(np.float64)
    scale = np.abs(W.reshape(M, K)) @ np.abs(x.astype(np.float64))
    assert np.max(np.abs(y - ref) / scale) < 2e-4


def test_matvec_float_rmsnorm_prologue(gpu):
    M, K = 300, 2048
    codes, scales, _ = _rand(M, K, 5)
    r = np.random.default_rng(6)
    x = r.normal(0, 3, K).astype(np.float32)
    w = r.uniform(0.8, 1.2, K).astype(np.float32)
    y = gpu.matvec_float(scales, codes, x, norm_w=w, eps=1e-6)
    xn = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    W = ((codes.astype(np.float64) - 1).reshape(M, -1, 128) * scales.astype(np.float64)[:, :, None]).reshape(M, K)
    assert np.max(np.abs(y - W @ xn) / (np.abs(W) @ np.abs(xn))) < 2e-4


def test_matvec_float_deterministic(gpu):
    """Two runs give bitwise identical results (no order-dependent atomics in the float path)."""
    codes, scales, _ = _rand(2048, 4096, 9)
    x = np.random.default_rng(1).normal(0, 1, 4096).astype(np.float32)
    a = gpu.matvec_float(scales, codes, x)
    b = gpu.matvec_float(scales, codes, x)
    assert np.array_equal(a, b)


def test_quantizer_matches_the_reference_fixture():
    """The GPU quantizer (trx_quantize_f_pow2) bit for bit against the reference's
    _quantize_f_pow2 outputs (tests/golden/golden_quant.npz) and the oracle on random vectors of
    the model widths."""
    import os
    from trixium_amd import bitexact
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_quant.npz"))
    for k in [k for k in z.files if k.startswith("q/") and k.endswith("/x")]:
        n = k[2:-2]
        q, e = bitexact.quantize_f_pow2(z[k])
        assert np.array_equal(q, z[f"q/{n}/x8"]) and e == int(z[f"q/{n}/e8"]), n
    r = np.random.default_rng(5)
    for K in (128, 2048, 4096, 12288, 17408):
        x = (r.standard_normal(K) * r.uniform(0.01, 50)).astype(np.float32)
        q, e = bitexact.quantize_f_pow2(x)
        wq, we = ob.quantize_f_pow2(x)
        assert np.array_equal(q, wq) and e == we, K


@pytest.mark.parametrize("kind", [L.KIND_TERNARY5, L.KIND_TERNARY])
def test_engine_projection_matches_the_reference_fixture(kind):
    """The projection through the engine (trx_gemv_ternary_quantized: quantize, exact matvec,
    scale by 2^(e8 + R - B)) bit for bit against the reference's mirror path
    (tests/golden/golden_quant.npz) and the oracle at the 8B widths."""
    import os
    import sys
    from trixium_amd import bitexact
    here = os.path.dirname(os.path.abspath(__file__))
    z = np.load(os.path.join(here, "golden", "golden_quant.npz"))
    sys.path.insert(0, os.path.join(here, "golden"))
    from make_golden_quant import projections
    for name, codes, scales, x in projections():
        y = bitexact.matvec_quantized(scales, codes, x, int(z[f"p/{name}/B"]), int(z[f"p/{name}/R"]), kind=kind)
        assert np.array_equal(y, z[f"p/{name}/y"]), name
    r = np.random.default_rng(9)
    for M, K in ((6144, 4096), (4096, 12288)):
        u = r.random((M, K))
        codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
        scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
        x = r.standard_normal(K).astype(np.float32)
        _, e16 = ob.fp16_decompose(scales)
        B = ob.choose_scale_bias(e16)
        R = ob.choose_result_shift(scales, B)
        x8, e8 = ob.quantize_f_pow2(x)
        want = ob.matvec_ternary(scales, codes, x8, B, R).astype(np.float32) * np.float32(2.0 ** (e8 + R - B))
        assert np.array_equal(bitexact.matvec_quantized(scales, codes, x, B, R, kind=kind), want)
