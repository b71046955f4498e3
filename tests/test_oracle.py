"""The CPU oracle pinned before it is trusted: the reference's known-answer tests restated, closed
forms and brute force on small cases, and the golden fixtures the reference produced."""

import hashlib

import numpy as np
import pytest

from oracle import bitexact as bx
from oracle.floatref import FloatRef
from trixium_amd import bons, configs as C, layout as L, synth


def test_rne_shift_known_answers():
    # test/model/test_bitexact.py:13-26 of the reference.
    assert bx.rne_shift(3, 1) == 2 and bx.rne_shift(1, 1) == 0 and bx.rne_shift(5, 1) == 2
    assert bx.rne_shift(7, 1) == 4 and bx.rne_shift(-1, 1) == 0 and bx.rne_shift(-3, 1) == -2
    assert bx.rne_shift(-5, 2) == -1 and bx.rne_shift(6, 2) == 2
    v = np.arange(-1000, 1000)
    for k in (1, 3, 7):
        assert np.array_equal(bx.rne_shift(v, k), np.rint(v / 2**k).astype(np.int64))


def test_fp16_decompose_exact():
    rng = np.random.default_rng(5)
    s = np.concatenate([rng.uniform(-1, 1, 1000).astype(np.float16),
                        np.array([0.0, 6e-8, -6e-8, 6e-5, 65504.0], np.float16)])
    m11, e16 = bx.fp16_decompose(s)
    assert np.array_equal(m11.astype(np.float64) * np.exp2(e16.astype(np.float64)), s.astype(np.float64))
    assert np.all(np.abs(m11) < 2048)


def test_matvec_ternary_accuracy_vs_float64():
    # test/model/test_bitexact.py:36-56: the only error is the per-group shift truncation.
    rng = np.random.default_rng(42)
    M, K = 64, 512
    scales = rng.uniform(0.01, 0.08, (M, K // 128)).astype(np.float16)
    codes = rng.integers(0, 3, (M, K), dtype=np.uint8)
    x8 = rng.integers(-127, 128, K, dtype=np.int8)
    _, e16 = bx.fp16_decompose(scales)
    B = bx.choose_scale_bias(e16)
    R = bx.choose_result_shift(scales, B)
    res = bx.matvec_ternary(scales, codes, x8, B, R)
    ref = (((codes.astype(np.float64) - 1) * x8).reshape(M, -1, 128).sum(2) * scales.astype(np.float64)).sum(1)
    got = res.astype(np.float64) * np.exp2(-B + R)
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-3)) < 1e-3


def test_matvec_ternary_bounds_hold_adversarial():
    # test/model/test_bitexact.py:58-70: K = 12288, all +1, x8 = 127, wide scale range.
    rng = np.random.default_rng(7)
    M, K = 16, 12288
    scales = (np.exp2(rng.uniform(-10, 0, (M, K // 128))) * 0.5).astype(np.float16)
    codes = np.full((M, K), 2, np.uint8)
    x8 = np.full(K, 127, np.int8)
    _, e16 = bx.fp16_decompose(scales)
    B = bx.choose_scale_bias(e16)
    res = bx.matvec_ternary(scales, codes, x8, B, bx.choose_result_shift(scales, B))
    assert res.dtype == np.int32


def test_matvec_ternary_brute_force_small():
    """Scalar evaluation of the engine rule on tiny shapes (a wrong shift direction or a
    dropped group fails here)."""
    rng = np.random.default_rng(11)
    for _ in range(20):
        M, G = 3, 2
        scales = np.exp2(rng.uniform(-16, 2, (M, G))).astype(np.float16) * rng.choice([-1, 1], (M, G)).astype(np.float16)
        codes = rng.integers(0, 3, (M, 128 * G), dtype=np.uint8)
        x8 = rng.integers(-127, 128, 128 * G, dtype=np.int8)
        B, R = 20, 3
        got = bx.matvec_ternary(scales, codes, x8, B, R)
        for m in range(M):
            acc = 0
            for g in range(G):
                gs = sum((int(codes[m, 128 * g + j]) - 1) * int(x8[128 * g + j]) for j in range(128))
                bits = int(scales[m, g].view(np.uint16))
                E, frac = (bits >> 10) & 31, bits & 1023
                m11 = (frac + 1024 if E else frac) * (-1 if bits & 0x8000 else 1)
                e16 = E - 25 if E else -24
                p = gs * m11
                acc += p << (e16 + B) if e16 + B >= 0 else p >> -(e16 + B)
            assert got[m] == acc >> R


def test_matvec_ternary_microbench_fixtures(golden):
    for (M, K) in C.MICROBENCH_SHAPES:
        r = np.random.default_rng(M * 7919 + K)
        u = r.random((M, K))
        codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
        scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
        x8 = r.integers(-127, 128, K, dtype=np.int8)
        g = golden[f"matvec/{M}x{K}"]
        _, e16 = bx.fp16_decompose(scales)
        B = bx.choose_scale_bias(e16)
        R = bx.choose_result_shift(scales, B)
        assert (B, R) == (g["B"], g["R"])
        res = bx.matvec_ternary(scales, codes, x8, B, R)
        assert hashlib.sha256(res.astype("<i4").tobytes()).hexdigest() == g["sha256"]
        assert res[:8].tolist() == g["head"]


def test_matvec_q8_accuracy():
    rng = np.random.default_rng(3)
    M, K = 32, 256
    scales = rng.uniform(0.005, 0.02, (M, K // 32)).astype(np.float16)
    q8w = rng.integers(-127, 128, (M, K), dtype=np.int8)
    x8 = rng.integers(-127, 128, K, dtype=np.int8)
    _, e16 = bx.fp16_decompose(scales)
    B = bx.choose_scale_bias(e16)
    R = bx.choose_result_shift(scales, B, gs_max=bx.GS_MAX_Q8)
    res = bx.matvec_q8(scales, q8w, x8, B, R)
    ref = ((q8w.astype(np.float64) * x8).reshape(M, -1, 32).sum(2) * scales.astype(np.float64)).sum(1)
    got = res.astype(np.float64) * np.exp2(-B + R)
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-2)) < 1e-3


def test_quantize_f_pow2_closed_form():
    x = np.array([0.5, -0.25, 1e-3, 0.0, -0.5], np.float32)
    q, e = bx.quantize_f_pow2(x)
    assert e == -7  # frexp(0.5) = (0.5, 0)
    assert q.tolist() == [64, -32, 0, 0, -64]
    q, e = bx.quantize_f_pow2(np.array([1.0, 0.0078125 * 1.5], np.float32))  # ties away from zero
    assert e == -6 and q.tolist() == [64, 1]
    assert bx.quantize_f_pow2(np.zeros(4, np.float32))[1] == 0


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid", "tiny-ternemb"])
def test_floatref_matches_fastref_fixture(tiny_images, golden, golden_arrays, name):
    """Step-wise oracle vs the reference's teacher-forced HybridRef: greedy tokens identical and
    logits within 1e-4 relative at the stored positions."""
    r = FloatRef(bons.BONSReader(tiny_images[(name, True)]))
    prompt = golden[f"prompt/{name}"]
    want = golden[f"fastref_tokens/{name}"]
    assert r.generate(prompt, len(want)) == want
    pos = golden_arrays[f"fastref_logits_pos/{name}"].tolist()
    ref = golden_arrays[f"fastref_logits/{name}"]
    r.reset()
    for i, t in enumerate(prompt + want):
        lg = r.step(t, want_logits=i in pos)
        if lg is not None:
            j = pos.index(i)
            assert np.abs(lg - ref[j]).max() <= 1e-4 * np.abs(ref[j]).max()


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid", "tiny-ternemb"])
def test_sequence_forward_matches_fastref_fixture(tiny_images, golden, golden_arrays, name):
    """The oracle's whole-sequence forward (FloatRef.prefill, the long-context tests' prompt pass)
    against the reference's teacher-forced HybridRef logits: at every stored position p the first
    p tokens run as two sequences (the second attending to the first's cache) and token p as a
    step, within 1e-4 of the fixture; and the state after a sequence equals the state after the
    same tokens stepped one by one (caches, conv windows, recurrent matrices, each within rounding)."""
    r = FloatRef(bons.BONSReader(tiny_images[(name, True)]))
    seq = golden[f"prompt/{name}"] + golden[f"fastref_tokens/{name}"]
    pos = golden_arrays[f"fastref_logits_pos/{name}"].tolist()
    ref = golden_arrays[f"fastref_logits/{name}"]
    for j, p in enumerate(pos):
        r.reset()
        a = p // 2
        if a:
            r.prefill(seq[:a])
        if p > a:
            r.prefill(seq[a:p])
        lg = r.step(seq[p])
        assert np.abs(lg - ref[j]).max() <= 1e-4 * np.abs(ref[j]).max(), p
        r.reset()
        lg = r.prefill(seq[:p + 1], want_logits=True)
        assert np.abs(lg - ref[j]).max() <= 1e-4 * np.abs(ref[j]).max(), p
    n = len(seq)
    a = FloatRef(bons.BONSReader(tiny_images[(name, True)]), kv_fp16=True)
    b = FloatRef(bons.BONSReader(tiny_images[(name, True)]), kv_fp16=True)
    a.prefill(seq)
    for t in seq:
        b.step(t, want_logits=False)
    assert a.pos == b.pos == n
    # fp16 values: a few fp16 steps apart at most where the fp32 sums round differently (a cache
    # row at the wrong position or out of order would be O(1) off).
    for l in a.k_cache:
        for ca, cb in ((a.k_cache[l], b.k_cache[l]), (a.v_cache[l], b.v_cache[l])):
            x, y = np.stack(ca), np.stack(cb)
            assert np.abs(x - y).max() <= 1e-3 * np.abs(y).max()
    for l in a.dn_state:
        assert np.abs(a.conv_state[l] - b.conv_state[l]).max() <= 1e-5
        assert np.abs(a.dn_state[l] - b.dn_state[l]).max() <= 1e-5 * max(1.0, np.abs(b.dn_state[l]).max())
    assert np.array_equal([int(np.argmax(a.step(t))) for t in (5, 9)], [int(np.argmax(b.step(t))) for t in (5, 9)])


def test_floatref_mirror_loop_contract(tiny_images, golden):
    """The hybrid mirror (exact) and the oracle agree; 2-bit and trit5 images give one model."""
    a = FloatRef(bons.BONSReader(tiny_images[("tiny-hybrid", True)]))
    b = FloatRef(bons.BONSReader(tiny_images[("tiny-hybrid", False)]))
    p = golden["prompt/tiny-hybrid"]
    assert a.generate(p, 8) == b.generate(p, 8) == golden["mirror_exact_tokens/tiny-hybrid"]


def test_shape_sample_steps_like_the_cpu_baseline():
    """The CPU baseline's sampled decode step (bench.py's cpu_baseline leg) runs on a small shape:
    a plain-basis reference with random weights and a filled KV cache, logits of the vocabulary."""
    from oracle.floatref import ShapeSample
    mc = C.TINY.replace(n_layer=2)
    s = ShapeSample(mc, 2, 20, seed=0)
    lg = s.step(1)
    assert lg.shape == (mc.vocab,) and np.isfinite(lg).all()
    s.step(2, want_logits=False)


def _yarn_fixture(tmp_path):
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from make_golden_yarn import SEED, yarn_config
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_yarn.npz"))
    cfg = yarn_config()
    p = str(tmp_path / "yarn.img")
    bons.write_image(cfg, synth.small_model_tensors(cfg, SEED, True), 1, p, trit5=True)
    return p, z


def test_yarn_rope_table_follows_floatmodel(tmp_path):
    """A YaRN-scaled model (factor 4 over an original context of 32) exists only in the image's
    rope table. The writer's image equals the reference writer's byte for byte (rope table
    included), and the oracle, rotating with the table's Q14 rows as the firmware and the mirror
    do, follows the reference's golden.FloatModel (float64 YaRN tables) to 1e-4 at positions on
    both sides of the original context, while fastref's plain RoPE is far from it: a table
    without the ramp or without mscale would fail one of the two."""
    import hashlib
    p, z = _yarn_fixture(tmp_path)
    assert hashlib.sha256(open(p, "rb").read()).hexdigest() == bytes(z["image_sha256"]).decode()
    img = bons.BONSReader(p)
    assert bons.image_rope_table(img) is not None
    r = FloatRef(img)
    seq, n = [int(t) for t in z["seq"]], int(z["n_prompt"])
    lg = [r.forward(seq[:n])] + [r.step(t) for t in seq[n:]]
    for i, pos in enumerate(z["pos"]):
        got, want = lg[pos - (n - 1)], z["floatmodel_logits"][i]
        assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max(), pos
        assert np.abs(z["fastref_logits"][i] - want).max() >= 0.1 * np.abs(want).max(), pos
        assert int(np.argmax(got)) == int(np.argmax(want))


def test_plain_rope_table_is_not_a_yarn_table(tiny_images):
    """Every fixture image carries a rope table; with yarn_factor 1 it is plain RoPE, which the
    loaders recognise (the oracle then computes the angles as fastref does)."""
    for key in (("tiny-qwen3", True), ("tiny-hybrid", False)):
        img = bons.BONSReader(tiny_images[key])
        assert img.find(L.ROLE_ROPE_TAB, 0) is not None
        assert bons.image_rope_table(img) is None


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid"])
def test_floatref_score_matches_fastref(tiny_images, name):
    """The oracle's score (next-token NLLs) and final normed hidden states against the reference's
    HybridRef.score on the same model and sequence (tests/golden/golden_score.npz)."""
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_score.npz"))
    r = FloatRef(bons.BONSReader(tiny_images[(name, True)]))
    nll, hid = r.score([int(t) for t in z[f"{name}/tokens"]])
    assert nll.shape == z[f"{name}/nll"].shape
    assert np.abs(nll - z[f"{name}/nll"]).max() <= 1e-4
    want = z[f"{name}/hidden"]
    got = hid[z[f"{name}/hidden_pos"]]
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()


def test_tensor_ref_equals_floatref_on_an_image(tmp_path):
    """TensorRef (the oracle over weights given as arrays, used at the headline shapes) steps like
    FloatRef over the same model written as an image: the hashed tiny model, its embedding from
    the ternary rows by the int16-table rule."""
    from oracle.floatref import TensorRef
    cfg = C.TINY.replace(name="tiny-hashed", n_layer=2, tie_embeddings=False, max_ctx=64)
    specs = synth.hashed_model_tensors(cfg, 4)
    p = str(tmp_path / "h.img")
    bons.write_image(cfg, specs, 1, p, trit5=True)
    a = FloatRef(bons.BONSReader(p), kv_fp16=True)
    w, g = {}, {}
    emb = None
    for s in specs:
        if L.is_ternary(s.kind):
            v = (s.values.astype(np.float32).reshape(s.rows, -1, 128) - 1) * s.scales.astype(np.float32)[:, :, None]
            w[(s.role, s.layer)] = v.reshape(s.rows, s.cols)
            if s.role == L.ROLE_TOK_EMB:
                emb = s
        else:
            g[(s.role, s.layer)] = s.values.reshape(-1).astype(np.float32)

    def row(t):
        m, e = bons.embed_bfp_rows(emb.values[t:t + 1], emb.scales[t:t + 1])
        return m[0].astype(np.float32) * np.float32(np.exp2(int(e[0])))

    b = TensorRef(cfg, w, g, row, kv_fp16=True)
    prompt = synth.random_prompt(cfg, 6, 4)
    for t in prompt:
        la, lb = a.step(t), b.step(t)
        assert np.abs(la - lb).max() <= 1e-5 * np.abs(la).max()
    assert a.generate([1, 2, 3], 5) == b.generate([1, 2, 3], 5)
    # The whole-sequence forward over the arrays (TensorRef.proj_many) equals FloatRef's.
    a.reset()
    b.reset()
    la, lb = a.prefill(prompt, want_logits=True), b.prefill(prompt, want_logits=True)
    assert np.abs(la - lb).max() <= 1e-5 * np.abs(la).max()


def test_quantizer_and_engine_projection_match_the_reference():
    """The oracle's quantize_f_pow2 and engine projection against the reference's
    model/mirror.py:45-51 and :663-678 on edge-case vectors (tests/golden/golden_quant.npz): ties
    away from zero, float32 lroundf (0.49999997 rounds to 1 there), a maximum at and just below a
    power of two, extreme magnitudes, a mantissa rounding to 128 and clipped, all zeros."""
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_quant.npz"))
    names = [k[2:-2] for k in z.files if k.startswith("q/") and k.endswith("/x")]
    assert len(names) >= 10
    for n in names:
        q, e = bx.quantize_f_pow2(z[f"q/{n}/x"])
        assert np.array_equal(q, z[f"q/{n}/x8"]) and e == int(z[f"q/{n}/e8"]), n
    assert z["q/ties/x8"].tolist() == [100, 3, -3, 4, -1, 1, -127, 127]
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from make_golden_quant import projections
    for name, codes, scales, x in projections():
        B, R = int(z[f"p/{name}/B"]), int(z[f"p/{name}/R"])
        x8, e8 = bx.quantize_f_pow2(x)
        y = bx.matvec_ternary(scales, codes, x8, B, R).astype(np.int32).astype(np.float32) * np.float32(2.0 ** (e8 + R - B))
        assert np.array_equal(y, z[f"p/{name}/y"]), name


def test_restored_row_exact_pinned():
    """The integer restore of a rotated embedding row (oracle restatement of model/bons.py:262-295)
    against an explicit Sylvester-matrix product in int64 (the value to within half an LSB of the
    result, so the butterfly order, the signs, the alignment to the smallest exponent and the
    normalisation are all fixed), and against the float restore that writes the int16 table rows
    (trixium_amd/hadamard.py:restored_bfp_rows, whose tables are byte-identical to the reference
    converter's) within one LSB; a zero row gives zeros and exponent 0."""
    from oracle import bitexact as ob
    from trixium_amd import hadamard as H
    r = np.random.default_rng(1)
    for hb, E in ((64, 256), (128, 512), (256, 1024), (1024, 2048)):
        i = np.arange(hb)
        Hm = np.where(np.bitwise_count((i[:, None] & i[None, :]).astype(np.uint64)) % 2 == 1, -1, 1).astype(np.int64)
        for t in range(6):
            codes = r.integers(0, 3, E).astype(np.uint8)
            sc = (r.uniform(0.001, 0.06, E // 128) * (2.0 ** r.integers(-6, 3, E // 128))).astype(np.float16)
            signs = np.where(r.random(E) < 0.5, -1, 1)
            m, e = ob.restored_row_exact(sc, codes, signs, hb)
            m11, e16 = ob.fp16_decompose(sc)
            emin = e16.min()
            v = ((codes.astype(np.int64).reshape(-1, 128) - 1) * (m11 * (2 ** (e16 - emin)))[:, None]).reshape(-1)
            y = np.concatenate([Hm @ v[b:b + hb] for b in range(0, E, hb)]) * signs
            want = y.astype(np.float64) * 2.0 ** (emin - (hb.bit_length() - 1) // 2)
            got = m.astype(np.float64) * 2.0 ** e
            assert 2 ** 14 <= np.abs(m.astype(np.int64)).max() <= 32767        # absmax in [2^14, 2^15)
            assert np.all(np.abs(got - want) <= 2.0 ** e * 0.5), (hb, t)
            mf, ef = H.restored_bfp_rows(sc[None], codes[None], signs, hb)
            gf = mf[0].astype(np.float64) * 2.0 ** ef[0]
            assert np.all(np.abs(gf - got) <= 2.0 ** max(e, int(ef[0])) * 1.0001), (hb, t)
    m, e = ob.restored_row_exact(np.full(2, 0.5, np.float16), np.ones(256, np.uint8), np.ones(256, np.int64), 64)
    assert e == 0 and not m.any()


def test_kv_ring_keeps_the_sinks_and_the_most_recent_positions(tiny_images, golden):
    """The oracle's KV ring (firmware/hybrid.c:170-181 kv_slot, every slot attended) against its
    specification: attention over the positions it keeps, [0, pin) and the last ctx_cap - pin, from
    a full cache (the same set in another order: equal to float rounding); and, with a window the
    sequence never leaves, the plain path exactly. A slot off by one keeps another position and
    fails the first comparison."""
    img = bons.BONSReader(tiny_images[("tiny-hybrid", True)])
    toks = golden["prompt/tiny-hybrid"] + golden["fastref_tokens/tiny-hybrid"]
    toks = (toks * 3)[:58]
    cap, pin = 20, 5

    def run(ring=None, window=False):
        r = FloatRef(img, kv_fp16=True)
        if ring:
            r.set_kv_ring(*ring, window=window)
        r.reset()
        return r, np.stack([r.step(t) for t in toks])

    r, ringed = run((cap, pin))
    assert r.kv_pin == pin
    assert all(len(r.k_cache[l]) == cap for l in r.k_cache)
    _, windowed = run((cap, pin), window=True)
    for i in range(len(toks)):
        err = np.abs(ringed[i] - windowed[i]).max() / np.abs(windowed[i]).max()
        assert err <= 1e-5, (i, err)
    _, plain = run()
    assert np.array_equal(ringed[:cap], plain[:cap])
    assert np.abs(ringed[cap + 8:] - plain[cap + 8:]).max() > 1e-3   # the ring forgets positions
    _, wide = run((len(toks), pin))
    assert np.array_equal(wide, plain)


def test_kv_ring_pin_is_clamped_as_the_firmware_clamps_it(tiny_images):
    """hybrid.c:1148-1149: at least the 4 sinks, at most a quarter of the window; no ring where the
    window holds at most twice the pin (kv_ring_on)."""
    r = FloatRef(bons.BONSReader(tiny_images[("tiny-hybrid", True)]))
    for cap, want_pin, got in ((64, 100, 16), (64, 0, 4), (64, 9, 9), (8, 4, 0), (9, 4, 4)):
        r.set_kv_ring(cap, want_pin)
        r.reset()
        assert r.kv_pin == got, (cap, want_pin, r.kv_pin)
