"""GGUF -> BONS conversion: the PrismML block codecs against hand-derived known answers and
the ggml C loops restated element by element, the GGUF reader against the files the writer
makes, and the converter against the images the reference's converter (model/convert.py) wrote
from the same synthetic GGUF files (tests/golden/golden_convert.json)."""

import hashlib
import json
import os

import numpy as np
import pytest

import synth_gguf
from synth_gguf import CASES, ROT_CASES
from trixium_amd import bons, configs as C, convert, gguf, hadamard as H, layout as L, qformats as Q

HERE = os.path.dirname(os.path.abspath(__file__))


def _sha(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


# Codecs -------------------------------------------------------------------------------------------

def test_q2_0_element_layout_and_values():
    """Weight j of a block is bits 2(j%4)..+1 of byte j/4 after the fp16 scale; w = (q - 1) d,
    code 3 included (dequantize_row_q2_0, element by element)."""
    rng = np.random.default_rng(42)
    codes = rng.integers(0, 4, (4, 128), dtype=np.uint8)
    scales = rng.uniform(0.001, 0.1, 4).astype(np.float16)
    raw = Q.q2_0_pack(scales, codes)
    assert raw.size == 4 * Q.BLOCK_Q2_0
    w = Q.q2_0_dequant(raw)
    for i in range(4):
        blk = raw[i * 34:(i + 1) * 34]
        d = np.float32(blk[:2].view(np.float16)[0])
        for j in range(128):
            q = (int(blk[2 + j // 4]) >> (2 * (j % 4))) & 3
            assert w[i * 128 + j] == np.float32((q - 1) * d)
    s2, c2 = Q.q2_0_unpack(raw)
    assert np.array_equal(s2, scales) and np.array_equal(c2, codes)
    one = np.ones((1, 128), np.uint8)
    one[0, 0], one[0, 1] = 0, 2
    w = Q.q2_0_dequant(Q.q2_0_pack(np.array([0.5], np.float16), one))
    assert w[0] == -0.5 and w[1] == 0.5 and not w[2:].any()


def test_ptq1_0_known_bytes():
    """Bytes worked out by hand from the format: 24 five-trit bytes in a run of 16 bytes (weights
    0..79, byte m of the run holding weights m, m+16, ..., m+64 as trits 0..4) then a run of 8
    (weights 80..119), two four-trit bytes (weights 120 + 2n + h), a byte being ceil(v 256 / 243)
    of its base-3 value v with trit 0 most significant."""
    def block(pos, code=1):
        c = np.zeros((1, 128), np.uint8)
        c[0, pos] = code
        return Q.ptq1_0_pack(np.array([1.0], np.float16), c)
    assert block(0)[0] == 86 and not block(0)[1:26].any()           # 81 -> ceil(81 256/243)
    assert block(16)[0] == 29                                         # trit 1 of byte 0: 27 -> 29
    assert block(64)[0] == 2                                          # trit 4: 1 -> ceil(256/243)
    assert block(15)[15] == 86 and block(80)[16] == 86 and block(88)[16] == 29
    assert block(87)[23] == 86 and block(120)[24] == 86 and block(121)[25] == 86
    assert block(122)[24] == 29 and block(127)[25] == 4               # qh trit 3: 3 -> ceil(768/243)
    twos = Q.ptq1_0_pack(np.array([1.0], np.float16), np.full((1, 128), 2, np.uint8))
    assert (twos[:24] == 255).all() and (twos[24:26] == 253).all()   # 242 -> 255; 240 -> 253
    assert twos[26:28].view(np.float16)[0] == 1.0
    for pos in (0, 16, 64, 15, 80, 88, 87, 120, 121, 122, 127):
        s, c = Q.ptq1_0_unpack(block(pos, 2))
        want = np.zeros(128, np.uint8)
        want[pos] = 2
        assert np.array_equal(c[0], want), pos


def test_ptq1_0_decodes_like_the_c_loop():
    """The vectorised decoder against dequantize_row_ptq1_0's loop restated scalar: runs of c in
    (32, 16, 8) bytes while they fit, trit n of byte q = ((q 3^n) & 255) 3 >> 8."""
    rng = np.random.default_rng(7)
    codes = rng.integers(0, 3, (37, 128), dtype=np.uint8)
    scales = rng.uniform(0.01, 0.1, 37).astype(np.float16)
    raw = Q.ptq1_0_pack(scales, codes)
    out = []
    for i in range(37):
        b = raw[i * 28:(i + 1) * 28]
        j = 0
        for c in (32, 16, 8):
            while j + c <= 24:
                for n in range(5):
                    for m in range(c):
                        out.append((((int(b[j + m]) * 3 ** n) & 255) * 3 >> 8))
                j += c
        for n in range(4):
            for h in range(2):
                out.append((((int(b[24 + h]) * 3 ** n) & 255) * 3 >> 8))
    assert np.array_equal(np.array(out, np.uint8), codes.reshape(-1))
    s2, c2 = Q.ptq1_0_unpack(raw)
    assert np.array_equal(s2, scales) and np.array_equal(c2, codes)
    assert np.array_equal(Q.ptq1_0_dequant(raw), Q.q2_0_dequant(Q.q2_0_pack(scales, codes)))


def test_q1_0_bits_and_ternary_bridge():
    rng = np.random.default_rng(9)
    bits = rng.integers(0, 2, (6, 128), dtype=np.uint8)
    scales = rng.uniform(0.001, 0.1, 6).astype(np.float16)
    raw = Q.q1_0_pack(scales, bits)
    assert raw.size == 6 * 18
    w = Q.q1_0_dequant(raw).reshape(6, 128)
    for i in (0, 5):
        for j in (0, 1, 7, 8, 127):
            bit = (int(raw[i * 18 + 2 + j // 8]) >> (j % 8)) & 1
            assert w[i, j] == (np.float32(scales[i]) if bit else -np.float32(scales[i]))
    s, c = Q.q1_0_to_ternary_codes(raw)
    assert np.array_equal(s, scales) and np.array_equal(c, bits * 2)


def test_q8_0_roundtrip_and_quant():
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, (16, 32), dtype=np.int8)
    s = rng.uniform(0.001, 0.1, 16).astype(np.float16)
    s2, q2 = Q.q8_0_unpack(Q.q8_0_pack(s, q))
    assert np.array_equal(s2, s) and np.array_equal(q2, q)
    w = rng.normal(0, 1, 128).astype(np.float32)
    assert np.abs(Q.q8_0_dequant(Q.q8_0_quant(w)) - w).max() < 0.02


def test_type_42_group_from_size():
    assert Q.q2_0_group(np.zeros(34 * 10, np.uint8), 1280) == 128
    assert Q.q2_0_group(np.zeros(18 * 20, np.uint8), 1280) == 64
    with pytest.raises(ValueError):
        Q.q2_0_group(np.zeros(100, np.uint8), 1280)


def test_bf16_is_the_top_half():
    x = np.array([1.0, -2.5, 3.140625], np.float32)
    top = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(Q.bf16_dequant(top.tobytes()), x)


# GGUF files ---------------------------------------------------------------------------------------

def test_gguf_reader_reads_what_the_writer_wrote(tmp_path):
    p = str(tmp_path / "t.gguf")
    a = np.arange(5, dtype=np.int32)
    md = {"general.architecture": "qwen3", "n": 7, "f": 1.5, "s": "text", "b": True,
          "arr": a, "strs": ["x", "yz"], "neg": gguf.Typed(gguf.T_I32, -3)}
    raw1 = Q.ptq1_0_pack(np.ones(3, np.float16), np.ones((3, 128), np.uint8))
    raw2 = np.arange(12, dtype=np.float32).tobytes()
    gguf.write_gguf(p, md, [("w", (3, 128), Q.GGML_PTQ1_0, raw1), ("v", (3, 4), Q.GGML_F32, raw2)])
    r = gguf.GGUFReader(p)
    assert r.metadata["n"] == 7 and r.metadata["f"] == 1.5 and r.metadata["s"] == "text"
    assert r.metadata["b"] is True and r.metadata["strs"] == ["x", "yz"] and r.metadata["neg"] == -3
    assert np.array_equal(r.metadata["arr"], a)
    w, v = r.tensors["w"], r.tensors["v"]
    assert (w.shape, w.type_name, w.nbytes, v.shape, v.type_name) == ((3, 128), "PTQ1_0", 84, (3, 4), "F32")
    assert (w.file_offset - r.data_start) % 32 == 0 and (v.file_offset - r.data_start) % 32 == 0
    assert np.array_equal(np.asarray(r.tensor_bytes("w")), raw1)
    assert np.array_equal(np.asarray(r.tensor_bytes("v")).view(np.float32), np.arange(12, dtype=np.float32))


def test_gguf_reader_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"XXXX" + bytes(20))
    with pytest.raises(ValueError, match="not a GGUF"):
        gguf.GGUFReader(str(p))
    good = str(tmp_path / "g.gguf")
    gguf.write_gguf(good, {"k": "v" * 40}, [])
    p.write_bytes(open(good, "rb").read()[:40])
    with pytest.raises(ValueError, match="truncated"):
        gguf.GGUFReader(str(p))


# The converter ------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def converted(tmp_path_factory):
    """Each golden case's GGUF, our image of it and the GGUF's ternary matrices."""
    d = tmp_path_factory.mktemp("convert")
    out = {}
    for c in CASES:
        g, img = str(d / (c["id"] + ".gguf")), str(d / (c["id"] + ".bons"))
        truth = synth_gguf.build(g, c["cfg"], c["seed"], c["arch"])
        convert.convert(g, c["channels"], img, kseg_max=c["kseg_max"], trit5=c["trit5"], check=True,
                        log=lambda *a: None)
        out[c["id"]] = (c, g, img, truth)
    return out


@pytest.mark.parametrize("case", [c["id"] for c in CASES])
def test_image_equals_the_reference_converters(converted, case):
    with open(os.path.join(HERE, "golden", "golden_convert.json")) as f:
        want = json.load(f)[case]
    c, g, img, _ = converted[case]
    assert _sha(g) == want["gguf_sha256"], "the synthetic GGUF changed: regenerate the fixture"
    assert _sha(img) == want["image_sha256"]


@pytest.mark.parametrize("case", [c["id"] for c in CASES])
def test_image_holds_the_gguf_weights(converted, case):
    """Every ternary matrix reads back as the GGUF's codes and scales (K-segments joined, padded
    vocabulary rows zero), the config is the metadata's, and the CRCs check."""
    c, g, img, truth = converted[case]
    r = bons.BONSReader(img)
    cfg = convert.config_from_gguf(gguf.GGUFReader(g))
    for k in ("n_layer", "n_embd", "n_head", "n_kv_head", "head_dim", "ffn_dim", "vocab", "layer_types",
              "dn_num_v_heads", "dn_num_k_heads", "dn_k_head_dim", "dn_v_head_dim", "dn_conv_kernel",
              "rope_dims", "attn_gated", "tie_embeddings"):
        assert getattr(cfg, k) == getattr(c["cfg"], k), k
    for name, (scales, codes) in truth.items():
        e = r.by_name[name] if name in r.by_name else r.by_name[name + ".k0"]
        parts = [r.entry_tensor(s) for s in r.ksegs(e)]
        s_img = np.concatenate([p[0] for p in parts], axis=1)
        v_img = np.concatenate([p[1] for p in parts], axis=1)
        rows = codes.shape[0]
        assert np.array_equal(v_img[:rows], codes) and np.array_equal(s_img[:rows], scales), name
        assert (v_img[rows:] == 1).all() and not s_img[rows:].any(), name
    assert convert.verify(img, log=lambda *a: None)


def test_verify_finds_a_corrupted_payload(converted, tmp_path):
    _, _, img, _ = converted["qwen3_ch1"]
    data = bytearray(open(img, "rb").read())
    r = bons.BONSReader(img)
    e = r.by_name["blk.1.ffn_up.weight"]
    data[r.header["payload_offset"] + e["chan_base_beats"] * L.BEAT + 5] ^= 0x10
    bad = tmp_path / "bad.bons"
    bad.write_bytes(bytes(data))
    assert not convert.verify(str(bad), log=lambda *a: None)


def test_beta_alpha_become_q8_rows(converted):
    """The hybrid's beta (Q8_0 in the file) is stored as it is; alpha (BF16) is requantised:
    amax/127 fp16 scales per 32 weights, values round-half-even, so it dequantises within half a
    step of the BF16 weights."""
    c, g, img, _ = converted["qwen35_hybrid_kseg"]
    r, gr = bons.BONSReader(img), gguf.GGUFReader(g)
    s, q = r.tensor("blk.0.ssm_beta.weight")
    s0, q0 = Q.q8_0_unpack(gr.tensor_bytes("blk.0.ssm_beta.weight"))
    assert np.array_equal(s.reshape(-1), s0) and np.array_equal(q.reshape(-1, 32), q0)
    s, q = r.tensor("blk.0.ssm_alpha.weight")
    w = Q.bf16_dequant(gr.tensor_bytes("blk.0.ssm_alpha.weight")).reshape(q.shape)
    step = np.repeat(s.astype(np.float32), 32, axis=1)
    assert np.all(np.abs(q * step - w) <= 0.5 * step * (1 + 1e-3) + 1e-7)


# PrismML rotation --------------------------------------------------------------------------------

def test_sylvester_matrix_and_restore():
    """H_2n = [[H_n, H_n], [H_n, -H_n]] with H_1 = [1]; R = H / sqrt(n) is orthonormal; restore
    undoes the fold z = R diag(s) e."""
    h = np.ones((1, 1), np.float32)
    while h.shape[0] < 256:
        h = np.block([[h, h], [h, -h]])
    assert np.array_equal(H.sign_matrix(256), h)
    R = H.matrix(256).astype(np.float64)
    assert np.allclose(R @ R.T, np.eye(256), atol=1e-6)
    rng = np.random.default_rng(0)
    s = np.where(rng.random(512) < 0.5, -1.0, 1.0).astype(np.float32)
    e = rng.normal(0, 1, (3, 512)).astype(np.float32)
    z = ((e * s).reshape(3, 2, 256) @ R.T.astype(np.float32)).reshape(3, 512)
    assert np.allclose(H.restore(z, s, 256), e, atol=1e-5)
    assert H.image_scales(1024) == (2.0 ** -5, 1.0) and H.image_scales(512) == (2.0 ** -4, 2.0 ** -0.5)
    assert H.image_gain(1024) == 1.0 and abs(H.image_gain(512) - np.sqrt(2)) < 1e-12


def test_restored_table_rows():
    """restored_bfp_rows: mantissas with the row absmax in [2^14, 2^15) whose value is the
    restored row times the image gain within half a mantissa step."""
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 3, (5, 256), dtype=np.uint8)
    scales = rng.uniform(0.01, 0.05, (5, 2)).astype(np.float16)
    s = np.where(rng.random(256) < 0.5, -1.0, 1.0).astype(np.float32)
    mant, exps = H.restored_bfp_rows(scales, codes, s, 128)
    z = ((codes.astype(np.float64) - 1).reshape(5, 2, 128) * scales.astype(np.float64)[:, :, None]).reshape(5, 256)
    e = H.restore(z.astype(np.float32), s, 128).astype(np.float64) * H.image_gain(128)
    amax = np.abs(mant.astype(np.int64)).max(axis=1)
    assert ((amax >= 2 ** 14 - 1) & (amax <= 32767)).all()
    assert np.all(np.abs(mant * 2.0 ** exps[:, None] - e) <= 0.5 * 2.0 ** exps[:, None] * (1 + 1e-6))


@pytest.fixture(scope="module")
def rotated(tmp_path_factory):
    d = tmp_path_factory.mktemp("rot")
    out = {}
    for c in ROT_CASES:
        g, img = str(d / (c["id"] + ".gguf")), str(d / (c["id"] + ".bons"))
        synth_gguf.build(g, c["cfg"], c["seed"], c["arch"], hadamard=c["hadamard"])
        convert.convert(g, c["channels"], img, kseg_max=c["kseg_max"], trit5=c["trit5"], log=lambda *a: None)
        out[c["id"]] = (c, g, img)
    return out


@pytest.mark.parametrize("case", [c["id"] for c in ROT_CASES])
def test_rotated_image_equals_the_reference_converters(rotated, case):
    """Rotation tensors, the odd-block fold and the restored embedding table, byte for byte."""
    with open(os.path.join(HERE, "golden", "golden_convert.json")) as f:
        want = json.load(f)[case]
    c, g, img = rotated[case]
    assert _sha(g) == want["gguf_sha256"], "the synthetic GGUF changed: regenerate the fixture"
    assert _sha(img) == want["image_sha256"]
    blk, scale, signs = H.image_rotation(bons.BONSReader(img))
    gg = gguf.GGUFReader(g)
    assert blk == c["hadamard"] and scale == H.image_scales(blk)[0]
    at = 0
    for w in gg.metadata["prism.hadamard.sign_widths"]:
        assert np.array_equal(signs[int(w)], gg.metadata["prism.hadamard.sign_values"][at:at + int(w)])
        at += int(w)


@pytest.mark.parametrize("case", [c["id"] for c in ROT_CASES])
def test_oracle_rotates_like_fastref(rotated, case):
    """The oracle's rotation (the image's rotation tensors before every ternary projection but
    beta/alpha) against the reference's HybridRef logits on the reference's image, every position
    of the prompt (tests/golden/golden_rot_logits.npz)."""
    from oracle.floatref import FloatRef
    z = np.load(os.path.join(HERE, "golden", "golden_rot_logits.npz"))
    prompt, want = [int(t) for t in z[case + "/prompt"]], z[case + "/logits"]
    ref = FloatRef(bons.BONSReader(rotated[case][2]))
    got = [ref.forward(prompt[:1])] + [ref.step(t) for t in prompt[1:]]
    for g, w in zip(got, want):
        assert np.max(np.abs(g - w)) <= 1e-4 * np.max(np.abs(w))
        assert np.argmax(g) == np.argmax(w)


def test_unsupported_inputs_are_errors(tmp_path):
    cfg = C.TINY.replace(name="t", n_layer=1)
    g = str(tmp_path / "g64.gguf")
    # A type-42 tensor in upstream's group-64 layout (18 bytes per 64 weights).
    md = synth_gguf._meta(cfg, "qwen3")
    gguf.write_gguf(g, md, [("token_embd.weight", (cfg.vocab, 256), Q.GGML_Q2_0, bytes(cfg.vocab * 4 * 18))])
    with pytest.raises(NotImplementedError, match="group-64"):
        convert.spec_from_gguf(gguf.GGUFReader(g), "token_embd.weight", 1, cfg.vocab)
    md["prism.hadamard.block_size"] = 256
    md["prism.hadamard.transform"] = "normalized-sylvester-walsh-hadamard"
    md["prism.hadamard.axis"] = "input-last-dimension"
    md["prism.hadamard.sign_widths"] = gguf.Typed(gguf.T_ARR, np.array([256], np.int32))
    md["prism.hadamard.sign_values"] = gguf.Typed(gguf.T_ARR, np.ones(256, np.int8))
    h = str(tmp_path / "had.gguf")
    gguf.write_gguf(h, md, [("token_embd.weight", (cfg.vocab, 256), Q.GGML_PQ2_0, bytes(cfg.vocab * 2 * 34))])
    assert convert.config_from_gguf(gguf.GGUFReader(h)).hadamard_block == 256
    md["prism.hadamard.axis"] = "output"
    gguf.write_gguf(h, md, [("token_embd.weight", (cfg.vocab, 256), Q.GGML_PQ2_0, bytes(cfg.vocab * 2 * 34))])
    with pytest.raises(ValueError, match="transform or axis"):
        convert.config_from_gguf(gguf.GGUFReader(h))


def test_command_line(converted, tmp_path, capsys):
    _, g, img, _ = converted["qwen3_ch1"]
    out = str(tmp_path / "cli.bons")
    assert convert.main(["convert", "--gguf", g, "--channels", "1", "--out", out]) == 0
    assert _sha(out) == _sha(img)
    assert json.load(open(str(tmp_path / "cli.json")))["n_channels"] == 1
    assert convert.main(["verify", "--image", out]) == 0
    convert.main(["inspect", g])
    assert "token_embd.weight" in capsys.readouterr().out


def test_split_wide_segments():
    """K-segments (model/bons.py:83-115): nseg = ceil(cols / kseg_max) ranges ending at group
    floor(G k / nseg), FLAG_KSEG with the index, the whole tensor's bias/rshift on every segment,
    and the pieces joining back to the tensor; Q8 capped at 255 code beats of 32 columns; the token
    embedding never split."""
    rng = np.random.default_rng(4)
    sc = rng.uniform(0.01, 0.05, (3, 40)).astype(np.float16)
    codes = rng.integers(0, 3, (3, 5120), dtype=np.uint8)
    t = bons.TensorSpec("w", L.ROLE_FFN_DOWN, 2, L.KIND_TERNARY, 3, 5120, scales=sc, values=codes)
    segs = bons.split_wide(t, 1536)
    assert [s.cols for s in segs] == [1280, 1280, 1280, 1280]           # 40 groups / 4 segments
    assert [s.kseg for s in segs] == [0, 1, 2, 3] and all(s.flags & L.FLAG_KSEG for s in segs)
    assert all((s.bias, s.rshift) == (t.bias, t.rshift) for s in segs)
    assert [s.name for s in segs] == ["w.k0", "w.k1", "w.k2", "w.k3"]
    assert np.array_equal(np.concatenate([s.values for s in segs], axis=1), codes)
    assert np.array_equal(np.concatenate([s.scales for s in segs], axis=1), sc)
    odd = bons.split_wide(t, 2000)                                        # 3 segments of 40 groups
    assert [s.cols for s in odd] == [13 * 128, 13 * 128, 14 * 128]
    lazy = bons.TensorSpec("w", L.ROLE_FFN_DOWN, 2, L.KIND_TERNARY, 3, 5120, scales=sc, loader=lambda: codes)
    assert np.array_equal(np.concatenate([s.load() for s in bons.split_wide(lazy, 1536)], axis=1), codes)
    q = rng.integers(-127, 128, (2, 16384), dtype=np.int8)
    q8 = bons.TensorSpec("b", L.ROLE_SSM_BETA, 0, L.KIND_Q8, 2, 16384,
                         scales=rng.uniform(0.01, 0.05, (2, 512)).astype(np.float16), values=q)
    # 16384 columns > 255 * 32 = 8160: 3 segments, edges at groups floor(512 k / 3) = 0, 170, 341, 512
    assert [s.cols for s in bons.split_wide(q8)] == [5440, 5472, 5472]
    emb = bons.TensorSpec("token_embd.weight", L.ROLE_TOK_EMB, 0, L.KIND_TERNARY, 3, 5120, scales=sc, values=codes)
    assert bons.split_wide(emb, 1536) == [emb]
