"""Batched prefill on the GPU (model/bitexact.py:121-125 matvec_ternary_rows, firmware/infer.c:
1956-1977 forward_pair: several prompt positions per weight pass).

- The multi-position GEMM (trx_gemm_ternary_f32) against float64 on trit5, 2-bit and Q8 rows:
  ragged row counts, odd group counts and a single group (the kernel's two 64-column steps),
  positions not a multiple of the block's 64, every epilogue, with and without the RMSNorm
  prologue.
- The decoder after a prefill against the fastref fixtures (greedy tokens) and the float oracle
  (logits at the last prompt position and at later teacher-forced positions), on the tiny
  models, the YaRN and rotated images and the 27B hybrid geometry; chunks of 1, 2 (shorter than
  the DeltaNet conv window), 5 and longer than the prompt; prefills that start mid-sequence.
- Two layers at the full Qwen3-8B width with the full LM head: the logits after a chunked
  prefill of an 80-token prompt within 2e-3 of the oracle and 16 greedy tokens identical.
"""

import ctypes

import numpy as np
import pytest

from oracle.floatref import FloatRef
from trixium_amd import _lib, bons, configs as C, layout as L, synth
from trixium_amd.bons import encode_rows

pytestmark = pytest.mark.gpu

KINDS = {"trit5": L.KIND_TERNARY5, "2bit": L.KIND_TERNARY, "q8": L.KIND_Q8}


def _rel_err(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / np.max(np.abs(ref)))


def _matrix(kind, M, K, rng):
    """Row packets and the float64 weights they hold (fp16 exactly as fastref caches them)."""
    if kind == L.KIND_Q8:
        q = rng.integers(-127, 128, (M, K), dtype=np.int8)
        sc = rng.uniform(0.01, 0.05, (M, K // 32)).astype(np.float16)
        w = (q.astype(np.float16).reshape(M, -1, 32) * sc[:, :, None]).astype(np.float16)
        return encode_rows(kind, K, sc, q), w.reshape(M, K).astype(np.float64)
    u = rng.random((M, K))
    codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
    if kind == L.KIND_TERNARY:
        codes[rng.random((M, K)) < 0.05] = 3                 # 2-bit code 3 is weight 2
    sc = rng.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
    w = (codes.astype(np.float64) - 1).reshape(M, -1, 128) * sc.astype(np.float64)[:, :, None]
    return encode_rows(kind, K, sc, codes), w.reshape(M, K)


def _gemm(rows, kind, M, K, x, norm_w, eps, epi, y0=None):
    n = x.shape[0]
    rb = _lib.DeviceBuffer.from_array(rows)
    xb = _lib.DeviceBuffer.from_array(x)
    gb = _lib.DeviceBuffer.from_array(norm_w) if norm_w is not None else None
    cols = M // 2 if epi == _lib.EPI_SWIGLU else M
    yb = _lib.DeviceBuffer.from_array(y0) if y0 is not None else _lib.DeviceBuffer(4 * n * cols)
    wb = _lib.DeviceBuffer(4 * n * (K + 1))
    _lib.call("trx_gemm_ternary_f32", rb.ptr, kind, M, K, xb.ptr, n, gb.ptr if gb else None, ctypes.c_float(eps),
              yb.ptr, epi, wb.ptr, None)
    _lib.call("trx_stream_sync", None)
    return yb.download(np.float32, n * cols).reshape(n, cols)


@pytest.mark.parametrize("kname", ["trit5", "2bit", "q8"])
@pytest.mark.parametrize("epi", [_lib.EPI_STORE, _lib.EPI_RESID, _lib.EPI_SWIGLU])
@pytest.mark.parametrize("M,K,n,norm", [(384, 256, 70, True), (200, 384, 5, False), (1024, 2048, 130, True),
                                        (6144, 2048, 64, False), (130, 128, 33, True)])
def test_gemm_matches_float64(kname, epi, M, K, n, norm):
    kind = KINDS[kname]
    rng = np.random.default_rng(M * 31 + K + n + epi)
    rows, W = _matrix(kind, M, K, rng)
    x = (rng.standard_normal((n, K)) * rng.uniform(0.5, 3.0, (n, 1))).astype(np.float32)
    g = rng.uniform(0.8, 1.2, K).astype(np.float32) if norm else None
    eps = 1e-6
    xd = x.astype(np.float64)
    if norm:
        xd = xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + eps) * g.astype(np.float64)
    ref, mag = xd @ W.T, np.abs(xd) @ np.abs(W).T
    y0 = rng.standard_normal((n, M)).astype(np.float32) if epi == _lib.EPI_RESID else None
    got = _gemm(rows, kind, M, K, x, g, eps, epi, y0).astype(np.float64)
    if epi == _lib.EPI_SWIGLU:
        F = M // 2
        gt, up = ref[:, :F], ref[:, F:]
        with np.errstate(over="ignore"):            # exp(-gt) = inf for large negative gt: silu -> 0
            want = gt / (1 + np.exp(-gt)) * up
        bound = 2e-5 * (mag[:, :F] * np.abs(up) + np.abs(gt) * mag[:, F:]) + 1e-7
    else:
        want = ref + (y0 if y0 is not None else 0)
        bound = 2e-5 * mag + 1e-6 * (np.abs(y0) if y0 is not None else 0) + 1e-7
    err = np.abs(got - want)
    print(kname, epi, M, K, n, "max err / bound", float(np.max(err / bound)))
    assert np.all(err <= bound)


@pytest.mark.parametrize("norm", [False, True])
def test_gemm_input_not_16_byte_aligned(norm):
    """x rows starting 4 bytes into a buffer take the input-plane kernel's 4-byte path; the result
    is held to the same float64 bound as the aligned calls."""
    kind, M, K, n = L.KIND_TERNARY5, 256, 512, 40
    rng = np.random.default_rng(17 + norm)
    rows, W = _matrix(kind, M, K, rng)
    x = rng.standard_normal((n, K)).astype(np.float32)
    g = rng.uniform(0.8, 1.2, K).astype(np.float32) if norm else None
    eps = 1e-6
    xd = x.astype(np.float64)
    if norm:
        xd = xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + eps) * g.astype(np.float64)
    ref, mag = xd @ W.T, np.abs(xd) @ np.abs(W).T
    rb = _lib.DeviceBuffer.from_array(rows)
    xb = _lib.DeviceBuffer(4 * (n * K + 1))
    xb.upload(x, offset=4)
    gb = _lib.DeviceBuffer.from_array(g) if norm else None
    yb = _lib.DeviceBuffer(4 * n * M)
    wb = _lib.DeviceBuffer(4 * n * (K + 1))
    _lib.call("trx_gemm_ternary_f32", rb.ptr, kind, M, K, xb.ptr + 4, n, gb.ptr if gb else None,
              ctypes.c_float(eps), yb.ptr, _lib.EPI_STORE, wb.ptr, None)
    _lib.call("trx_stream_sync", None)
    got = yb.download(np.float32, n * M).reshape(n, M).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2e-5 * mag + 1e-7)


@pytest.mark.parametrize("epi", [_lib.EPI_STORE, _lib.EPI_SWIGLU])
@pytest.mark.parametrize("norm", [False, True])
def test_gemm_large_inputs_stay_finite(epi, norm):
    """Rows with values past fp16's range (1e5, 3e9; with the RMSNorm prologue, gains of 1e6):
    the planes of such a row are scaled by a power of two and the result scaled back, so the
    GEMM equals float64 within the same bound as for small inputs, and no output is inf or NaN
    (an unscaled fp16 plane would turn a 1e5 input into inf - inf = NaN for every output)."""
    kind, M, K, n = L.KIND_TERNARY5, 256, 512, 6
    rng = np.random.default_rng(17 + epi + 2 * norm)
    rows, W = _matrix(kind, M, K, rng)
    x = rng.standard_normal((n, K)).astype(np.float32)
    x[1, 7] = 1.0e5
    x[3, :] *= 3.0e9
    x[4, 100] = -65520.0
    g = rng.uniform(0.8, 1.2, K).astype(np.float32) if norm else None
    if norm:
        g[5] = 1.0e6
    eps = 1e-6
    xd = x.astype(np.float64)
    if norm:
        xd = xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + eps) * g.astype(np.float64)
    ref, mag = xd @ W.T, np.abs(xd) @ np.abs(W).T
    got = _gemm(rows, kind, M, K, x, g, eps, epi).astype(np.float64)
    assert np.isfinite(got).all()
    if epi == _lib.EPI_SWIGLU:
        F = M // 2
        gt, up = ref[:, :F], ref[:, F:]
        with np.errstate(over="ignore"):
            want = gt / (1 + np.exp(-gt)) * up
        bound = 2e-5 * (mag[:, :F] * np.abs(up) + np.abs(gt) * mag[:, F:]) + 1e-7
    else:
        want, bound = ref, 2e-5 * mag + 1e-7
    err = np.abs(got - want)
    print("large inputs", epi, norm, "max err / bound", float(np.max(err / bound)))
    assert np.all(err <= bound)


def test_gemm_refuses_bad_arguments():
    wb = _lib.DeviceBuffer(4096)
    with pytest.raises(_lib.TrxError):
        _lib.call("trx_gemm_ternary_f32", wb.ptr, L.KIND_TERNARY5, 4, 200, wb.ptr, 1, None, ctypes.c_float(1e-6),
                  wb.ptr, _lib.EPI_STORE, wb.ptr, None)          # K not a multiple of 128
    with pytest.raises(_lib.TrxError):
        _lib.call("trx_gemm_ternary_f32", wb.ptr, L.KIND_F16, 4, 128, wb.ptr, 1, None, ctypes.c_float(1e-6),
                  wb.ptr, _lib.EPI_STORE, wb.ptr, None)          # not a ternary or Q8 kind


# Decoder ----------------------------------------------------------------------------------------

N_NEW = {"tiny-qwen3": 64, "tiny-ternemb": 32, "tiny-hybrid": 24}


def _decoder(path, **kw):
    from trixium_amd.model import Decoder
    return Decoder.from_image(path, **kw)


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-ternemb", "tiny-hybrid"])
@pytest.mark.parametrize("chunk", [1, 2, 5, 64])
def test_prefill_generates_the_fastref_tokens(tiny_images, golden, name, chunk):
    """generate_fresh with the prompt prefilled (15 positions in chunks, then the last prompt
    position as a step): the fixture's greedy tokens, both row formats."""
    prompt = golden[f"prompt/{name}"]
    ref = golden[f"fastref_tokens/{name}"][:N_NEW[name]]
    for t5 in (True, False):
        dec = _decoder(tiny_images[(name, t5)], max_new=N_NEW[name], prefill_chunk=chunk)
        assert dec.generate_fresh(prompt, N_NEW[name]) == ref, (t5, chunk)
        dec.close()


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid"])
def test_prefill_state_matches_the_oracle(tiny_images, golden, name):
    """Logits after a prefill and at later positions within 2e-3 of the oracle, with prefills that
    start mid-sequence (attention over earlier cache rows, the DeltaNet state and conv window
    carried over): forward(prompt[:7]) then forward(prompt[7:]) then forward(5 tokens)."""
    prompt = golden[f"prompt/{name}"]
    extra = golden[f"fastref_tokens/{name}"][:5]
    p = tiny_images[(name, True)]
    ref = FloatRef(bons.BONSReader(p), kv_fp16=True)
    for chunk in (3, 64):
        dec = _decoder(p, prefill_chunk=chunk)
        ref.reset()
        errs = []
        for piece in (prompt[:7], prompt[7:], extra):
            got = dec.forward(piece)
            want = None
            for i, t in enumerate(piece):
                want = ref.step(t, want_logits=i == len(piece) - 1)
            errs.append(_rel_err(got, want))
        print(name, "chunk", chunk, "rel errs", errs)
        assert max(errs) <= 2e-3
        # The decoder moves on from the prefilled state like one that stepped every position.
        d1 = _decoder(p)
        d1.forward(prompt)
        dec.reset()
        dec.forward(prompt)
        assert _rel_err(dec.forward([extra[0]]), d1.forward([extra[0]])) <= 2e-3
        dec.close()
        d1.close()


def test_prefill_refuses_positions_that_compute_logits(tiny_images, golden):
    prompt = golden["prompt/tiny-qwen3"]
    dec = _decoder(tiny_images[("tiny-qwen3", True)])
    dec.reset()
    dec.feed(prompt)
    with pytest.raises(_lib.TrxError):
        dec.prefill(len(prompt))                 # the last fed position computes logits
    with pytest.raises(_lib.TrxError):
        dec.prefill(len(prompt) + 3)             # past the fed tokens
    dec.prefill(len(prompt) - 1)
    dec.step(1)
    assert np.isfinite(dec.logits()).all()


def test_prefill_buffers_do_not_grow_with_every_prompt(tiny_images):
    """A session whose prompts keep growing: the prefill buffers grow in powers of two and the
    smaller ones are freed, so the device bytes stay within the buffers of twice the longest
    chunk, and the logits stay those of a fresh decoder."""
    from trixium_amd.model import INFO_DEVICE_BYTES
    path = tiny_images[("tiny-qwen3", True)]
    dec = _decoder(path, prefill_chunk=1024, max_ctx=128)
    base = dec.info(INFO_DEVICE_BYTES)
    sizes = []
    for n in range(2, 120, 7):
        dec.reset()
        dec.forward(list(range(1, n + 1)))
        sizes.append(dec.info(INFO_DEVICE_BYTES) - base)
    # tiny-qwen3: at most 128 rows of 256-wide activations, FFN 768, q|k|v 512, and the sums of a
    # small GEMM's K parts (16 x 128 floats a row): a few MB.
    per_row = 4 * 256 + 2 * 2 * 768 + 4 + 4 + 4 * 512 + 4 * 256 + 4 * 768 + 4 * 256 + 4 * 16 * 128
    assert max(sizes) <= 128 * per_row, sizes
    assert sizes[-1] == max(sizes)
    ref = _decoder(path, prefill_chunk=1024, max_ctx=128)
    lg = ref.forward(list(range(1, 114)))
    dec.reset()
    assert _rel_err(dec.forward(list(range(1, 114))), lg) <= 1e-6
    dec.close()
    ref.close()


def test_prefill_yarn_image(tmp_path):
    """The YaRN image (RoPE from the image's Q14 table): the reference's FloatModel greedy tokens
    after a prefilled prompt."""
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from make_golden_yarn import SEED, yarn_config
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_yarn.npz"))
    cfg = yarn_config()
    p = str(tmp_path / "yarn.img")
    bons.write_image(cfg, synth.small_model_tensors(cfg, SEED, True), 1, p, trit5=True)
    seq, n = [int(t) for t in z["seq"]], int(z["n_prompt"])
    dec = _decoder(p, max_new=len(seq) - n, prefill_chunk=4)
    assert dec.generate_fresh(seq[:n], len(seq) - n) == seq[n:]


@pytest.mark.parametrize("case", ["qwen3_rot128", "qwen35_rot256"])
def test_prefill_rotated_image(tmp_path, case):
    """PrismML-rotated images (the rotation in the GEMM's input planes; the DeltaNet beta/alpha
    unrotated): logits after a prefilled prompt within 2e-3 of the oracle and the reference's
    HybridRef logits within 1e-2 (tests/golden/golden_rot_logits.npz)."""
    import os
    import synth_gguf
    from trixium_amd import convert
    c = next(x for x in synth_gguf.ROT_CASES if x["id"] == case)
    g, p = str(tmp_path / "m.gguf"), str(tmp_path / "m.bons")
    synth_gguf.build(g, c["cfg"], c["seed"], c["arch"], hadamard=c["hadamard"])
    convert.convert(g, 1, p, trit5=c["trit5"], log=lambda *a: None)
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_rot_logits.npz"))
    prompt, want = [int(t) for t in z[case + "/prompt"]], z[case + "/logits"]
    ref = FloatRef(bons.BONSReader(p), kv_fp16=True)
    dec = _decoder(p, prefill_chunk=3)
    got = dec.forward(prompt)
    assert _rel_err(got, ref.forward(prompt)) <= 2e-3
    assert _rel_err(got, want[-1]) <= 1e-2
    dec.reset()
    d2 = _decoder(p)
    assert dec.generate(prompt, 6) == d2.generate(prompt, 6)


def test_prefill_hybrid_27b_geometry(tmp_path):
    """A Gated DeltaNet layer and a gated attention layer at the 27B hybrid's geometry: logits
    after the prefilled prompt and at every generated position within 2e-3 of the reference's
    fastref logits, and its greedy tokens."""
    import hashlib
    import os
    fx = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_h_geometry.npz"))
    cfg = C.QWEN35_27B.replace(name="qwen3.5-27b-geometry-2l", n_layer=2, layer_types=("deltanet", "attn"),
                               vocab=512, max_ctx=64)
    p = str(tmp_path / "h.img")
    bons.write_image(cfg, synth.small_model_tensors(cfg, 7, True), 1, p, trit5=True)
    assert hashlib.sha256(open(p, "rb").read()).hexdigest() == bytes(fx["image_sha256"]).decode()
    prompt, tokens = [int(t) for t in fx["prompt"]], [int(t) for t in fx["tokens"]]
    dec = _decoder(p, max_new=8, prefill_chunk=2)
    lg = [dec.forward(prompt)] + [dec.forward([t]) for t in tokens]
    errs = [_rel_err(g, w) for g, w in zip(lg, fx["logits"])]
    print("27B geometry with prefill, rel errs", errs)
    assert max(errs) <= 2e-3
    assert dec.generate_fresh(prompt, len(tokens)) == tokens


@pytest.mark.timeout(900)
def test_prefill_full_width_8b_matches_the_oracle():
    """Two layers at the full Qwen3-8B width with the full 151936-row LM head: an 80-token prompt
    prefilled in chunks of 32 (the last chunk ragged), the logits at its last position within 2e-3
    of the oracle, then 16 greedy tokens identical to the oracle's."""
    from test_headline_gpu import _oracle
    from trixium_amd.model import Decoder
    mc = C.QWEN3_8B.replace(name="qwen3-8b-shape-2l", n_layer=2, max_ctx=128)
    seed = 23
    dec = Decoder.synthetic(mc, seed, weight_kind=L.KIND_TERNARY5, max_new=16, prefill_chunk=32)
    ref = _oracle(dec, mc, seed)
    prompt = synth.random_prompt(mc, 80, seed)
    got = dec.forward(prompt)
    want = None
    for i, t in enumerate(prompt):
        want = ref.step(t, want_logits=i == len(prompt) - 1)
    err = _rel_err(got, want)
    print("8B width prefill: last prompt position rel err", err, flush=True)
    assert err <= 2e-3
    ids, lg = [], want
    for i in range(16):
        ids.append(int(np.argmax(lg)))
        if i + 1 < 16:
            lg = ref.step(ids[-1])
    assert dec.generate_fresh(prompt, 16) == ids
