"""The GPU token loop against the golden fixtures (model/fastref.py greedy tokens and logits) and
the float oracle: tiny Qwen3 (fp16 embedding table, F16 head), tiny ternary-embedding Qwen3
(tied trit5 head), tiny hybrid (Gated DeltaNet + gated attention), both row formats, sharded
images, eager vs hipGraph, and the counter-based device generator."""

import numpy as np
import pytest

from oracle.floatref import FloatRef
from trixium_amd import bons, configs as C, layout as L, synth
from trixium_amd._lib import TrxError

pytestmark = pytest.mark.gpu

# Logits tolerance: max |gpu - ref| <= LOGIT_RTOL * max |ref| per position. The GPU quantises
# each GEMV input to int16 per 128-group and caches K/V in fp16; the fixture is fp32 throughout.
LOGIT_RTOL = 1e-2
N_NEW = {"tiny-qwen3": 64, "tiny-ternemb": 32, "tiny-hybrid": 24}


def _decoder(path, **kw):
    from trixium_amd.model import Decoder
    return Decoder.from_image(path, **kw)


def _rel_err(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / np.max(np.abs(ref)))


def _teacher_forced_logits(dec, seq, n_prompt):
    """Logits at positions n_prompt-1 .. len(seq)-1 with the given tokens fed."""
    dec.reset()
    out = [dec.forward(seq[:n_prompt])]
    for t in seq[n_prompt:]:
        out.append(dec.forward([t]))
    return np.stack(out)


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-ternemb", "tiny-hybrid"])
def test_logits_match_fastref_fixture(tiny_images, golden, golden_arrays, name):
    prompt = golden[f"prompt/{name}"]
    seq = prompt + golden[f"fastref_tokens/{name}"]
    dec = _decoder(tiny_images[(name, True)])
    lg = _teacher_forced_logits(dec, seq, len(prompt))
    pos = golden_arrays[f"fastref_logits_pos/{name}"]
    ref = golden_arrays[f"fastref_logits/{name}"]
    for i, p in enumerate(pos):
        err = _rel_err(lg[p - (len(prompt) - 1)], ref[i])
        print(f"{name} pos {p}: rel err {err:.2e}")
        assert err <= LOGIT_RTOL, (name, p, err)


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-ternemb", "tiny-hybrid"])
def test_greedy_tokens_match_fastref(tiny_images, golden, name):
    prompt = golden[f"prompt/{name}"]
    ref = golden[f"fastref_tokens/{name}"]
    dec = _decoder(tiny_images[(name, True)], max_new=N_NEW[name])
    got = dec.generate_fresh(prompt, N_NEW[name])
    assert got == ref[:N_NEW[name]]


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid"])
def test_logits_match_oracle_every_position(tiny_images, golden, name):
    """Every position of a teacher-forced run against the float oracle with an fp16 KV cache."""
    prompt = golden[f"prompt/{name}"]
    seq = prompt + golden[f"fastref_tokens/{name}"][:12]
    img = bons.BONSReader(tiny_images[(name, True)])
    dec = _decoder(tiny_images[(name, True)])
    lg = _teacher_forced_logits(dec, seq, len(prompt))
    ref = FloatRef(img, kv_fp16=True)
    want = [ref.forward(prompt)] + [ref.step(t) for t in seq[len(prompt):]]
    errs = [_rel_err(g, w) for g, w in zip(lg, want)]
    print(name, "max rel err", max(errs))
    assert max(errs) <= 2e-3


def test_graph_replay_equals_eager(tiny_images, golden):
    name = "tiny-hybrid"
    prompt = golden[f"prompt/{name}"]
    a = _decoder(tiny_images[(name, True)], max_new=16)
    b = _decoder(tiny_images[(name, True)], max_new=16)
    ta = a.generate_fresh(prompt, 16, use_graph=True)
    tb = b.generate_fresh(prompt, 16, use_graph=False)
    assert ta == tb
    assert np.array_equal(a.logits(), b.logits())
    assert np.array_equal(a.hidden(), b.hidden())
    # A second replay sequence on the same graph after a reset gives the same result.
    assert a.generate_fresh(prompt, 16, use_graph=True) == ta
    assert np.array_equal(a.logits(), b.logits())


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid"])
def test_two_bit_rows_match_trit5(tiny_images, golden, name):
    prompt = golden[f"prompt/{name}"]
    a = _decoder(tiny_images[(name, True)])
    b = _decoder(tiny_images[(name, False)])
    assert b.cfg.weight_kind == L.KIND_TERNARY and a.cfg.weight_kind == L.KIND_TERNARY5
    # Same integer group sums; the float combine may run in another order per format, and fp16
    # rounding of the cached K/V turns 1e-7 differences into ~1e-4 ones over the prompt.
    la, lb = a.forward(prompt), b.forward(prompt)
    assert _rel_err(la, lb) <= 1e-3
    assert int(np.argmax(la)) == int(np.argmax(lb))


def test_sharded_image_loads_the_same_model(tmp_path, tiny_images, golden):
    name, cfg = "tiny-hybrid", C.TINY_HYBRID
    p2 = str(tmp_path / "n2.img")
    bons.write_image(cfg, synth.small_model_tensors(cfg, 1, True), 2, p2, trit5=True)
    prompt = golden[f"prompt/{name}"]
    a = _decoder(tiny_images[(name, True)], max_new=8)
    b = _decoder(p2, max_new=8)
    assert a.generate_fresh(prompt, 8) == b.generate_fresh(prompt, 8)
    assert np.array_equal(a.logits(), b.logits())


def test_forward_in_pieces_equals_one_forward(tiny_images, golden):
    name = "tiny-qwen3"
    prompt = golden[f"prompt/{name}"]
    d = _decoder(tiny_images[(name, True)])
    whole = d.forward(prompt)
    assert d.position() == len(prompt) - 1
    d.reset()
    assert d.position() == -1
    d.forward(prompt[:5])
    d.forward(prompt[5:11])
    parts = d.forward(prompt[11:])
    assert np.array_equal(whole, parts)
    # generate() continues from the current position (FloatModel.generate).
    cont = d.generate([int(np.argmax(parts))], 4)
    d.reset()
    ref = d.generate(prompt + [int(np.argmax(parts))], 4)
    assert cont == ref


def test_context_limit_is_an_error(tiny_images, golden):
    d = _decoder(tiny_images[("tiny-qwen3", True)], max_ctx=32, max_new=8)
    prompt = golden["prompt/tiny-qwen3"]
    with pytest.raises(TrxError):
        d.generate_fresh(prompt, 20)          # 16 + 20 - 1 positions > 32
    with pytest.raises(TrxError):
        d.forward(list(range(33)))
    with pytest.raises(TrxError):
        d.forward([d.vocab])                  # token out of range
    assert d.generate_fresh(prompt, 8) == golden["fastref_tokens/tiny-qwen3"][:8]


def test_device_generator_matches_host_hash(tmp_path):
    """The counter-based weights filled in HBM equal the host hash, byte for byte, and the model
    they make decodes like the oracle run on the same tensors written as a BONS image (the
    embedding decoded from the ternary rows on the device, from the int16 table in the oracle)."""
    from trixium_amd.model import Decoder
    cfg = C.TINY.replace(name="tiny-hashed", n_layer=2, tie_embeddings=False, max_ctx=64)
    seed = 11
    specs = synth.hashed_model_tensors(cfg, seed)
    dec = Decoder.synthetic(cfg, seed, weight_kind=L.KIND_TERNARY5, max_new=16)
    for s in specs:
        got = dec.read_tensor(s.role, s.layer)
        if s.kind == L.KIND_TERNARY:
            want = bons.encode_rows(L.KIND_TERNARY5, s.cols, s.scales, s.values)
        else:
            want = s.values.astype(np.float32).view(np.uint8)
        assert np.array_equal(got, np.asarray(want).reshape(-1)), s.name
    p = str(tmp_path / "hashed.img")
    bons.write_image(cfg, specs, 1, p, trit5=True)
    ref = FloatRef(bons.BONSReader(p), kv_fp16=True)
    prompt = synth.random_prompt(cfg, 8, seed)
    lg = dec.forward(prompt)
    want = ref.forward(prompt)
    assert _rel_err(lg, want) <= 2e-3
    for t in (3, 1000, 7):
        assert _rel_err(dec.forward([t]), ref.step(t)) <= 2e-3


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-ternemb", "tiny-hybrid"])
@pytest.mark.parametrize("packed,tf", [(0, 0), (63, 0), (63, 63)])
@pytest.mark.parametrize("t5", [True, False])
def test_packed_projections_match_oracle(tiny_images, golden, name, packed, tf, t5):
    """Every projection on the packed GEMV (63 = TRX_PACK_ALL), with the per-block table or with
    the table-free lookups (tf 63), or none of them, on trit5 and 2-bit images: logits at every
    position against the float oracle and the greedy tokens against the fixture."""
    from trixium_amd.model import Decoder
    prompt = golden[f"prompt/{name}"]
    seq = prompt + golden[f"fastref_tokens/{name}"][:12]
    img = bons.BONSReader(tiny_images[(name, t5)])
    dec = Decoder.from_image(tiny_images[(name, t5)], max_new=N_NEW[name], packed_ops=packed, table_free_ops=tf)
    assert dec.packed_ops == packed and dec.table_free_ops == tf
    lg = _teacher_forced_logits(dec, seq, len(prompt))
    ref = FloatRef(img, kv_fp16=True)
    want = [ref.forward(prompt)] + [ref.step(t) for t in seq[len(prompt):]]
    errs = [_rel_err(g, w) for g, w in zip(lg, want)]
    print(name, packed, tf, t5, "max rel err", max(errs))
    assert max(errs) <= 2e-3
    got = dec.generate_fresh(prompt, N_NEW[name])
    assert got == golden[f"fastref_tokens/{name}"][:N_NEW[name]]


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid"])
def test_taps_of_the_last_forward(tiny_images, golden, name):
    """The intermediate vectors (q|k|v of the last attention layer, its attention output, the
    last layer's SwiGLU activation) after a forward, with the packed GEMVs handing their partial
    sums on (the attention sums the q|k|v partials and keeps the rows) and with the row-packet
    kernel (which stores each projection): the same vectors within the int16 activations'
    rounding, and the q|k|v rows equal to the oracle's projection of the last attention layer."""
    from trixium_amd.model import Decoder
    prompt = golden[f"prompt/{name}"]
    taps = []
    for packed in (63, 0):
        dec = Decoder.from_image(tiny_images[(name, True)], max_new=4, packed_ops=packed)
        dec.forward(prompt)
        taps.append(dec.taps())
        dec.close()
    for k in ("qkv", "attn", "act"):
        assert np.abs(taps[0][k]).max() > 0, k
        assert _rel_err(taps[0][k], taps[1][k]) <= 2e-3, k
    # The oracle's q|k|v of the last attention layer at the last prompt position.
    img = bons.BONSReader(tiny_images[(name, True)])
    ref = FloatRef(img, kv_fp16=True)
    ref.forward(prompt[:-1])
    la = max(l for l in range(ref.n_layer) if not ref.dn[l])
    seen = {}
    orig = ref.attention

    def spy(l, hn, pos):
        if l == la:
            seen["qkv"] = np.concatenate([ref.proj(r, l, hn) for r in (L.ROLE_ATTN_Q, L.ROLE_ATTN_K, L.ROLE_ATTN_V)])
        return orig(l, hn, pos)

    ref.attention = spy
    ref.step(prompt[-1])
    assert _rel_err(taps[0]["qkv"], seen["qkv"]) <= 2e-3


def test_packed_graph_replay_equals_eager(tiny_images, golden):
    from trixium_amd.model import Decoder
    name = "tiny-hybrid"
    prompt = golden[f"prompt/{name}"]
    a = Decoder.from_image(tiny_images[(name, True)], max_new=16, packed_ops=63, use_graph=True)
    b = Decoder.from_image(tiny_images[(name, True)], max_new=16, packed_ops=63, use_graph=False)
    assert a.generate_fresh(prompt, 16) == b.generate_fresh(prompt, 16)
    a.reset(); b.reset()
    assert np.array_equal(a.forward(prompt), b.forward(prompt))


def test_packed_path_at_full_width():
    """Two layers at Qwen3-1.7B width (2048 wide, ffn 6144, the 151936-row head): row tiles in
    the hundreds, all projections sharing one packed workspace. Every projection on the packed
    GEMV against none of them (the row-packet path, itself checked against the oracle above):
    logits within the int16 activation rounding of the row-packet path, same greedy tokens."""
    from trixium_amd.model import Decoder
    cfg = C.QWEN3_1P7B.replace(name="qwen3-1.7b-width-2l", n_layer=2, max_ctx=128)
    prompt = synth.random_prompt(cfg, 24, 3)
    a = Decoder.synthetic(cfg, 5, weight_kind=L.KIND_TERNARY5, max_new=16, packed_ops=0)
    b = Decoder.synthetic(cfg, 5, weight_kind=L.KIND_TERNARY5, max_new=16, packed_ops=63)
    assert a.packed_ops == 0 and b.packed_ops == 63
    la, lb = a.forward(prompt), b.forward(prompt)
    errs = [_rel_err(lb, la)]
    for t in (17, 90000, 5):
        errs.append(_rel_err(b.forward([t]), a.forward([t])))
    print("full width packed vs row-packet rel err", errs)
    assert max(errs) <= 2e-3
    a.reset(); b.reset()
    ta, tb = a.generate_fresh(prompt, 16), b.generate_fresh(prompt, 16)
    n = next((i for i, (x, y) in enumerate(zip(ta, tb)) if x != y), len(ta))
    assert n >= 8, (ta, tb)


@pytest.fixture(scope="module")
def h_geometry_image(tmp_path_factory):
    """The two-layer 27B-hybrid-geometry model of tests/golden/make_golden_h.py, written by this
    repository's writer (its sha256 is the reference writer's, checked below)."""
    import hashlib
    import os
    fx = dict(np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_h_geometry.npz")))
    cfg = C.QWEN35_27B.replace(name="qwen3.5-27b-geometry-2l", n_layer=2, layer_types=("deltanet", "attn"),
                               vocab=512, max_ctx=64)
    p = str(tmp_path_factory.mktemp("h") / "h.img")
    print("writing the 27B-geometry image", flush=True)
    bons.write_image(cfg, synth.small_model_tensors(cfg, 7, True), 1, p, trit5=True)
    sha = hashlib.sha256(open(p, "rb").read()).hexdigest()
    assert sha == bytes(fx["image_sha256"]).decode()
    return p, fx


@pytest.mark.parametrize("packed", [-1, 0])
def test_hybrid_27b_geometry_matches_fixture(h_geometry_image, packed):
    """A Gated DeltaNet layer and a gated attention layer at the 27B hybrid's geometry (width
    5120, 24 q / 4 kv heads of 256 with 64 RoPE dims, 48 v / 16 k DeltaNet heads of 128, FFN
    17408): logits at the last prompt position and every generated one within 2e-3 of the
    reference's fastref logits, and its greedy tokens, with the library's kernel choice (-1) and
    with every projection on the row-packet kernel (0)."""
    from trixium_amd.model import Decoder
    p, fx = h_geometry_image
    prompt, tokens = [int(t) for t in fx["prompt"]], [int(t) for t in fx["tokens"]]
    dec = Decoder.from_image(p, max_new=8, packed_ops=packed)
    lg = _teacher_forced_logits(dec, prompt + tokens, len(prompt))
    errs = [_rel_err(g, w) for g, w in zip(lg, fx["logits"])]
    print("27B geometry, packed", dec.packed_ops, "rel errs", errs)
    assert max(errs) <= 2e-3
    assert dec.generate_fresh(prompt, len(tokens)) == tokens


@pytest.mark.parametrize("case", ["qwen3_ch1", "qwen35_hybrid_kseg"])
def test_converted_gguf_decodes_like_the_oracle(tmp_path, case):
    """A synthetic Bonsai GGUF (PTQ1_0/PQ2_0/Q2_0/Q1_0 ternary blocks, Q8_0 and BF16 DeltaNet head
    projections) converted to a trit5 image decodes on the GPU like the oracle reads the image."""
    import synth_gguf
    from trixium_amd import convert
    c = next(x for x in synth_gguf.CASES if x["id"] == case)
    g, p = str(tmp_path / "m.gguf"), str(tmp_path / "m.bons")
    synth_gguf.build(g, c["cfg"], c["seed"], c["arch"])
    convert.convert(g, 1, p, kseg_max=c["kseg_max"], trit5=True, log=lambda *a: None)
    prompt = synth.random_prompt(c["cfg"], 8, c["seed"])
    dec = _decoder(p)
    ref = FloatRef(bons.BONSReader(p), kv_fp16=True)
    assert _rel_err(dec.forward(prompt), ref.forward(prompt)) <= 2e-3
    for t in (5, 700, 11, 42):
        assert _rel_err(dec.forward([t]), ref.step(t)) <= 2e-3


@pytest.mark.parametrize("case", ["qwen3_rot128", "qwen35_rot256"])
def test_rotated_image_decodes_like_fastref(tmp_path, case):
    """A PrismML-rotated model (rotation tensors, folded weights, restored embedding table) on the
    GPU: the fast Walsh-Hadamard transform before every projection against the oracle's rotation
    tensors on the same image, and against the reference's HybridRef logits on the reference
    converter's image (tests/golden/golden_rot_logits.npz), every prompt position."""
    import os
    import synth_gguf
    from trixium_amd import convert
    c = next(x for x in synth_gguf.ROT_CASES if x["id"] == case)
    g, p = str(tmp_path / "m.gguf"), str(tmp_path / "m.bons")
    synth_gguf.build(g, c["cfg"], c["seed"], c["arch"], hadamard=c["hadamard"])
    convert.convert(g, 1, p, trit5=c["trit5"], log=lambda *a: None)
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_rot_logits.npz"))
    prompt, want = [int(t) for t in z[case + "/prompt"]], z[case + "/logits"]
    dec = _decoder(p)
    ref = FloatRef(bons.BONSReader(p), kv_fp16=True)
    got = [dec.forward(prompt[:1])] + [dec.forward([t]) for t in prompt[1:]]
    oracle = [ref.forward(prompt[:1])] + [ref.step(t) for t in prompt[1:]]
    for gl, o, w in zip(got, oracle, want):
        assert _rel_err(gl, o) <= 2e-3
        assert _rel_err(gl, w) <= LOGIT_RTOL
        assert np.argmax(gl) == np.argmax(w)
    dec.reset()
    toks = dec.generate(prompt, 6)
    dec2 = _decoder(p, use_graph=False)
    assert toks == dec2.generate(prompt, 6)


@pytest.mark.parametrize("block", [512, 1024])
def test_rotation_in_the_gemv_prologue(tmp_path, block):
    """Rotation blocks wider than the packed GEMV's 256-column slice: every GEMV block transforms
    the whole rotation block holding its slice. The packed path (rotation in the GEMV prologue)
    against the oracle's rotation tensors and against the row-packet path (a separate rotation
    launch), every position of a teacher-forced run."""
    from trixium_amd import hadamard as H
    cfg = C.TINY.replace(name="rot-wide", n_layer=2, n_embd=1024, n_head=8, n_kv_head=2, head_dim=128,
                         ffn_dim=2048, vocab=512, max_ctx=64, tie_embeddings=False)
    rng = np.random.default_rng(block)
    signs = {w: tuple(int(v) for v in np.where(rng.random(w) < 0.5, -1, 1)) for w in (1024, 2048)}
    rcfg = cfg.replace(hadamard_block=block, hadamard_signs=signs)
    specs = synth.small_model_tensors(cfg, 9, fp16_embedding=False) + H.rotation_specs(rcfg)
    p = str(tmp_path / "rot.bons")
    bons.write_image(rcfg, specs, 1, p, trit5=True)
    prompt = synth.random_prompt(cfg, 6, 9)
    ref = FloatRef(bons.BONSReader(p), kv_fp16=True)
    want = [ref.forward(prompt[:1])] + [ref.step(t) for t in prompt[1:]]
    for packed in (-1, 0):
        dec = _decoder(p, packed_ops=packed)
        got = [dec.forward(prompt[:1])] + [dec.forward([t]) for t in prompt[1:]]
        for g, w in zip(got, want):
            assert _rel_err(g, w) <= 2e-3, (packed, _rel_err(g, w))


def test_synthetic_hybrid_decodes():
    """A synthetic hybrid (device-generated ternary and float tensors, host Q8 beta|alpha rows):
    finite logits, and the graph replay generates what eager launches generate."""
    from trixium_amd.model import Decoder
    mc = C.TINY_HYBRID.replace(max_ctx=64)
    a = Decoder.synthetic(mc, 3, max_new=16)
    b = Decoder.synthetic(mc, 3, max_new=16, use_graph=False)
    prompt = synth.random_prompt(mc, 8, 3)
    assert np.isfinite(a.forward(prompt)).all()
    a.reset()
    assert a.generate(prompt, 8) == b.generate(prompt, 8)
    assert np.array_equal(a.read_tensor(L.ROLE_SSM_BETA, 1), b.read_tensor(L.ROLE_SSM_BETA, 1))


def test_yarn_rope_table_decodes_like_floatmodel(tmp_path):
    """A YaRN-scaled model (its scaling lives only in the image's rope table) on the GPU: the
    attention rotates with the table's Q14 rows. Every teacher-forced position within 2e-3 of the
    oracle, the reference's golden.FloatModel logits (tests/golden/golden_yarn.npz) within 1e-2,
    and FloatModel's 80 greedy tokens."""
    import os
    import sys
    from trixium_amd.model import Decoder
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from make_golden_yarn import SEED, yarn_config
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_yarn.npz"))
    cfg = yarn_config()
    p = str(tmp_path / "yarn.img")
    bons.write_image(cfg, synth.small_model_tensors(cfg, SEED, True), 1, p, trit5=True)
    seq, n = [int(t) for t in z["seq"]], int(z["n_prompt"])
    dec = Decoder.from_image(p, max_new=len(seq) - n)
    assert dec.cfg.rope_table == 1
    lg = _teacher_forced_logits(dec, seq, n)
    ref = FloatRef(bons.BONSReader(p), kv_fp16=True)
    want = [ref.forward(seq[:n])] + [ref.step(t) for t in seq[n:]]
    errs = [_rel_err(g, w) for g, w in zip(lg, want)]
    print("yarn: max rel err vs oracle", max(errs))
    assert max(errs) <= 2e-3
    for i, pos in enumerate(z["pos"]):
        assert _rel_err(lg[pos - (n - 1)], z["floatmodel_logits"][i]) <= LOGIT_RTOL
    assert dec.generate_fresh(seq[:n], len(seq) - n) == seq[n:]


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid"])
def test_score_hidden_and_head_match_fastref(tiny_images, name):
    """Decoder.score / hidden / logits(Hs) (model/fastref.py:244-273) on the GPU: the next-token
    NLLs and the final normed hidden states against the reference's HybridRef.score
    (tests/golden/golden_score.npz) and the oracle; hidden() after a forward is that position's
    normed state; the LM head applied to the returned states gives the decode's own logits."""
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_score.npz"))
    toks = [int(t) for t in z[f"{name}/tokens"]]
    dec = _decoder(tiny_images[(name, True)])
    nll, hid = dec.score(toks)
    ref_nll, ref_hid = FloatRef(bons.BONSReader(tiny_images[(name, True)]), kv_fp16=True).score(toks)
    print(name, "nll err vs fastref", np.abs(nll - z[f"{name}/nll"]).max(), "vs oracle", np.abs(nll - ref_nll).max())
    assert np.abs(nll - ref_nll).max() <= 2e-3
    assert np.abs(nll - z[f"{name}/nll"]).max() <= 2e-2
    assert _rel_err(hid, ref_hid) <= 2e-3
    hp = z[f"{name}/hidden_pos"]
    assert _rel_err(hid[hp], z[f"{name}/hidden"]) <= LOGIT_RTOL
    # hidden() of the last forward, and the head over given hidden states.
    dec.reset()
    lg = dec.forward(toks[:20])
    assert np.allclose(dec.hidden(), hid[19], rtol=0, atol=1e-5 * np.abs(hid[19]).max())
    proj = dec.logits(hid[[19, 5]])
    assert proj.shape == (2, dec.vocab)
    assert _rel_err(proj[0], lg) <= 1e-4
    assert _rel_err(dec.logits(dec.hidden()[None])[0], lg) <= 1e-4


@pytest.mark.parametrize("case", ["qwen3_rot128", "qwen35_rot256"])
def test_rotated_image_without_the_int16_table(tmp_path, case):
    """A rotated image converted without the int16 embedding table (`--no-emb16`): every token's
    row is restored to the plain basis in integers on the GPU (the firmware's embed_row_restore,
    model/bons.py:262-295). Logits at every prompt position within 2e-3 of the oracle's (which
    restores the rows with its own restatement), within 1e-2 of the same model with the table
    (whose rows differ by at most one LSB), the same tokens; eager, graph and the batched prefill
    agree."""
    import synth_gguf
    from trixium_amd import convert
    c = next(x for x in synth_gguf.ROT_CASES if x["id"] == case)
    g, p, p16 = str(tmp_path / "m.gguf"), str(tmp_path / "m.bons"), str(tmp_path / "m16.bons")
    synth_gguf.build(g, c["cfg"], c["seed"], c["arch"], hadamard=c["hadamard"])
    convert.convert(g, 1, p, trit5=c["trit5"], emb16=False, log=lambda *a: None)
    convert.convert(g, 1, p16, trit5=c["trit5"], log=lambda *a: None)
    img = bons.BONSReader(p)
    assert img.find(L.ROLE_TOK_EMB16, 0) is None
    prompt = synth.random_prompt(c["cfg"], 8, c["seed"])
    dec = _decoder(p)
    assert dec.cfg.emb_mode == 2
    ref = FloatRef(img, kv_fp16=True)
    d16 = _decoder(p16)
    got = [dec.forward(prompt[:1])] + [dec.forward([t]) for t in prompt[1:]]
    want = [ref.forward(prompt[:1])] + [ref.step(t) for t in prompt[1:]]
    w16 = [d16.forward(prompt[:1])] + [d16.forward([t]) for t in prompt[1:]]
    for gl, o, t16 in zip(got, want, w16):
        assert _rel_err(gl, o) <= 2e-3
        assert _rel_err(gl, t16) <= 1e-2
    dec.reset()
    toks = dec.generate(prompt, 6)
    assert toks == _decoder(p, use_graph=False).generate(prompt, 6)
    assert toks == _decoder(p, prefill_chunk=3).generate(prompt, 6)
