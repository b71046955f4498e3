"""BONS format layer (trixium_amd.layout / bons): the reference's known answers, round trips, and
byte identity with images the reference writer produced from the same tensors."""

import hashlib
import os

import numpy as np
import pytest

from trixium_amd import layout as L, bons, configs as C, synth


def test_beat_math_known_answers():
    # test/model/test_layout.py:17-24 of the reference.
    assert L.code_beats(4096, L.KIND_TERNARY) == 32
    assert L.scale_beats(4096, L.KIND_TERNARY) == 2
    assert L.row_beats(2048, L.KIND_TERNARY) == 17
    assert L.code_beats(2048, L.KIND_Q8) == 64
    assert L.scale_beats(2048, L.KIND_Q8) == 4


@pytest.mark.parametrize("K,b2,b5", [(2048, 544, 448), (4096, 1088, 896), (6144, 1632, 1344),
                                     (12288, 3264, 2688), (17408, 4640, 3840)])
def test_row_bytes(K, b2, b5):
    G = K // 128
    assert L.row_bytes(K, L.KIND_TERNARY) == 32 * (-(-G // 16) + G) == b2
    assert L.row_bytes(K, L.KIND_TERNARY5) == 32 * (-(-G // 16) + -(-26 * G // 32)) == b5


def test_header_and_entry_roundtrip():
    hdr = L.pack_header(C.TINY_HYBRID, 2, 25, 1000, 0xDEADBEEF, b"\x01" * 32)
    assert len(hdr) == L.HEADER_SIZE
    h = L.unpack_header(hdr)
    assert (h["n_layer"], h["n_channels"], h["payload_beats"]) == (4, 2, 1000)
    assert h["table_crc32"] == 0xDEADBEEF and h["tokenizer_sha256"] == b"\x01" * 32
    assert h["layer_types"] == C.TINY_HYBRID.layer_types
    assert (h["dn_num_v_heads"], h["rope_dims"], h["attn_gated"]) == (8, 16, 1)
    e = L.pack_entry(L.ROLE_FFN_GATE, L.KIND_TERNARY, 0, 5, 512, 256, 123, 456, 0xCAFEBABE,
                     bias=26, rshift=7, name="blk.5.ffn_gate.weight")
    d = L.unpack_entry(e)
    assert len(e) == L.ENTRY_SIZE
    assert (d["role"], d["layer"], d["rows"], d["cols"], d["group"]) == (L.ROLE_FFN_GATE, 5, 512, 256, 128)
    assert (d["chan_base_beats"], d["chan_len_beats"], d["bias"], d["rshift"]) == (123, 456, 26, 7)
    assert d["name"] == "blk.5.ffn_gate.weight"
    # Names longer than 24 bytes are truncated (the field is fixed).
    assert L.unpack_entry(L.pack_entry(0, 0, 0, 10, 1, 128, 0, 0, 0, name="blk.10.ffn_down.weight.k1"))["name"] == "blk.10.ffn_down.weight.k"


def test_trit5_decode_table_known_answer():
    """Every byte value decodes to five base-3 digits, LSB digit first (the known answer of the
    reference's test_trit5.test_decode_table: packing then unpacking 128 random codes)."""
    rng = np.random.default_rng(1)
    for _ in range(50):
        codes = rng.integers(0, 3, (1, 128)).astype(np.uint8)
        packed = bons.trit5_pack(codes)
        assert packed.shape == (1, 26)
        digits = []
        for b in packed[0]:
            v = int(b)
            for _k in range(5):
                digits.append(v % 3)
                v //= 3
        assert digits[:128] == codes[0].tolist() and digits[128:] == [0, 0]
        assert np.array_equal(bons.trit5_unpack(packed, 128), codes)
    assert bons.trit5_pack(np.full((1, 128), 2, np.uint8)).max() == 242


@pytest.mark.parametrize("kind", [L.KIND_TERNARY, L.KIND_TERNARY5])
def test_row_codec_roundtrip(kind):
    rng = np.random.default_rng(3)
    for K in (128, 384, 2048):
        codes = rng.integers(0, 3, (7, K)).astype(np.uint8)
        scales = rng.uniform(0.01, 0.05, (7, K // 128)).astype(np.float16)
        pk = bons.encode_rows(kind, K, scales, codes)
        assert pk.shape == (7, L.row_bytes(K, kind))
        s, v = bons.decode_rows(kind, K, pk)
        assert np.array_equal(v, codes) and np.array_equal(s, scales)


@pytest.mark.parametrize("name,seed,fp,cfg", [("tiny-qwen3", 0, True, C.TINY), ("tiny-hybrid", 1, True, C.TINY_HYBRID)])
@pytest.mark.parametrize("trit5", [True, False])
@pytest.mark.parametrize("nch", [1, 2])
def test_image_bytes_match_reference_writer(tmp_path, golden, name, seed, fp, cfg, trit5, nch):
    p = str(tmp_path / "m.img")
    bons.write_image(cfg, synth.small_model_tensors(cfg, seed, fp), nch, p, trit5=trit5)
    with open(p, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == golden[f"image_sha256/{cfg.name}/trit5={int(trit5)}/n{nch}"]


def test_ternary_embedding_image_matches_reference_writer(tmp_path, golden):
    p = str(tmp_path / "m.img")
    bons.write_image(C.TINY, synth.small_model_tensors(C.TINY, 3, False), 1, p, trit5=True)
    with open(p, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == golden["image_sha256/tiny-ternemb/trit5=1/n1"]


def test_reader_recovers_tensors_across_channels(tmp_path):
    specs = synth.small_model_tensors(C.TINY, 0, True)
    p = str(tmp_path / "m.img")
    bons.write_image(C.TINY, synth.small_model_tensors(C.TINY, 0, True), 2, p, trit5=True)
    r = bons.BONSReader(p)
    for s in specs:
        sc, v = r.tensor(s.name)
        assert np.array_equal(v, s.values.astype(v.dtype)), s.name
        if s.scales is not None:
            assert np.array_equal(sc, s.scales)
    # rope table, .w16 companions and the embedding table exist.
    assert "rope_tab" in r.by_name and "blk.0.attn_norm.w16" in r.by_name
    assert r.find(L.ROLE_TOK_EMB16) is not None


def test_embed_bfp_rows_matches_reference_fixture(golden_arrays):
    m, e = bons.embed_bfp_rows(golden_arrays["emb16_codes"], golden_arrays["emb16_scales"])
    assert np.array_equal(m, golden_arrays["emb16_mant"])
    assert np.array_equal(e, golden_arrays["emb16_exp"])


def test_embed_bfp_rows_scalar_form():
    """A scalar statement of the same integer rule (the reference's test_bons scalar check):
    align each group to the row's smallest exponent, normalise the live absmax to 15 bits."""
    rng = np.random.default_rng(9)
    codes = rng.integers(0, 3, (20, 256)).astype(np.uint8)
    scales = np.exp2(rng.uniform(-14, 4, (20, 2))).astype(np.float16)
    codes[3, :128] = 1
    from trixium_amd.fixedpoint import fp16_split
    m, e = bons.embed_bfp_rows(codes, scales)
    for r in range(20):
        m11, e16 = fp16_split(scales[r])
        emin = int(e16.min())
        sh = [min(int(x) - emin, 20) for x in e16]
        amax = max([abs(int(m11[g])) << sh[g] for g in range(2) if (codes[r, 128 * g:128 * (g + 1)] != 1).any()] or [0])
        k2 = amax.bit_length() - 15
        row = []
        for g in range(2):
            for c in codes[r, 128 * g:128 * (g + 1)]:
                v = (int(c) - 1) * int(m11[g])
                n = sh[g] - k2
                row.append(v << n if n >= 0 else v >> -n)
        assert np.array_equal(m[r], np.array(row, dtype=np.int64).astype(np.int16))
        assert e[r] == emin + k2


def test_hashed_generator_statistics():
    codes = synth.hashed_codes(0, 7, np.arange(64), 4096)
    frac = np.bincount(codes.reshape(-1), minlength=3) / codes.size
    assert abs(frac[0] - 0.3) < 0.01 and abs(frac[1] - 0.4) < 0.01 and abs(frac[2] - 0.3) < 0.01
    s = synth.hashed_scales(0, 7, np.arange(64), 4096).astype(np.float32)
    assert s.min() >= 0.01 and s.max() <= 0.05 and abs(s.mean() - 0.03) < 0.002
    # Rows are independent of which other rows are generated.
    assert np.array_equal(synth.hashed_codes(0, 7, np.array([5, 9]), 4096), codes[[5, 9]])
    assert not np.array_equal(synth.hashed_codes(1, 7, np.array([5]), 4096), codes[[5]])
