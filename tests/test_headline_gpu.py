"""The headline shapes on the GPU against the float oracle.

Two layers at the full Qwen3-8B width (4096 wide, FFN 12288, 32 q / 8 kv heads of 128, the
untied 151936-row ternary LM head) and at the full Qwen3-1.7B width (2048 wide, FFN 6144, the
tied 151936-row ternary embedding as the head), with every weight from the device generator; and
one Gated DeltaNet plus one gated attention layer at the full Qwen3.5-27B width with its
248320-row head.
The oracle runs on the weights read back from HBM (a sample of rows of every tensor checked
against the host hash first): every prompt position's logits within 2e-3 and the first 64 greedy
tokens identical. At full depth (36 and 28 layers) the checks are size-independent properties:
graph replay bitwise equal to eager launches, the packed GEMV against the row-packet GEMV, and
finite logits.
"""

import numpy as np
import pytest

from oracle.floatref import TensorRef
from trixium_amd import bons, configs as C, layout as L, synth

pytestmark = pytest.mark.gpu

TRIT5 = L.KIND_TERNARY5
N_PROMPT, N_GREEDY = 32, 64


def _rel_err(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / np.max(np.abs(ref)))


def _dequant(raw, rows, cols, chunk=8192):
    """BONS trit5 rows (bytes) -> float32 (code - 1) * scale, in row chunks."""
    rb = L.row_bytes(cols, TRIT5)
    raw = np.asarray(raw, np.uint8).reshape(-1)[:rows * rb].reshape(rows, rb)
    out = np.empty((rows, cols), np.float32)
    for r0 in range(0, rows, chunk):
        sc, codes = bons.decode_rows(TRIT5, cols, raw[r0:r0 + chunk])
        w = (codes.astype(np.float32).reshape(codes.shape[0], -1, 128) - 1.0) * sc.astype(np.float32)[:, :, None]
        out[r0:r0 + chunk] = w.reshape(codes.shape[0], cols)
    return out, raw


def _check_rows(raw, rows, cols, seed, role, layer, rng, n=4):
    """A few rows of a device-generated tensor against the host hash, byte for byte."""
    rb = L.row_bytes(cols, TRIT5)
    rr = np.sort(rng.choice(rows, size=n, replace=False))
    tid = synth.tensor_id(role, layer)
    want = bons.encode_rows(TRIT5, cols, synth.hashed_scales(seed, tid, rr, cols), synth.hashed_codes(seed, tid, rr, cols))
    assert np.array_equal(raw[rr], np.asarray(want).reshape(n, rb)), (role, layer)


def _oracle(dec, mc, seed):
    """TensorRef over the weights in HBM (rows checked against the host hash)."""
    rng = np.random.default_rng(seed)
    E, hd, F, V = mc.n_embd, mc.head_dim, mc.ffn_dim, mc.vocab
    shapes = {L.ROLE_ATTN_Q: (mc.n_head * hd, E), L.ROLE_ATTN_K: (mc.n_kv_head * hd, E),
              L.ROLE_ATTN_V: (mc.n_kv_head * hd, E), L.ROLE_ATTN_OUT: (E, mc.n_head * hd),
              L.ROLE_FFN_GATE: (F, E), L.ROLE_FFN_UP: (F, E), L.ROLE_FFN_DOWN: (E, F)}
    weights, gains = {}, {}
    for l in range(mc.n_layer):
        for role, (r, c) in shapes.items():
            w, raw = _dequant(dec.read_tensor(role, l), r, c)
            _check_rows(raw, r, c, seed, role, l, rng)
            weights[(role, l)] = w
        for role, n in ((L.ROLE_ATTN_NORM, E), (L.ROLE_FFN_NORM, E), (L.ROLE_ATTN_Q_NORM, hd), (L.ROLE_ATTN_K_NORM, hd)):
            g = dec.read_tensor(role, l).view(np.float32)[:n].copy()
            want = synth.hashed_uniform(seed, synth.tensor_id(role, l), 3, np.arange(n), synth.GAIN_LO, synth.GAIN_HI)
            assert np.array_equal(g, want), (role, l)
            gains[(role, l)] = g
    gains[(L.ROLE_OUT_NORM, 0)] = dec.read_tensor(L.ROLE_OUT_NORM, 0).view(np.float32)[:E].copy()
    emb_raw = np.asarray(dec.read_tensor(L.ROLE_TOK_EMB, 0)).reshape(-1)
    rb = L.row_bytes(E, TRIT5)
    emb_raw = emb_raw[:V * rb].reshape(V, rb)
    _check_rows(emb_raw, V, E, seed, L.ROLE_TOK_EMB, 0, rng)
    if mc.tie_embeddings:
        weights[(L.ROLE_TOK_EMB, 0)], _ = _dequant(emb_raw, V, E)
    else:
        w, raw = _dequant(dec.read_tensor(L.ROLE_LM_HEAD, 0), V, E)
        _check_rows(raw, V, E, seed, L.ROLE_LM_HEAD, 0, rng)
        weights[(L.ROLE_LM_HEAD, 0)] = w

    def embed_row(tok):
        sc, codes = bons.decode_rows(TRIT5, E, emb_raw[tok:tok + 1])
        mant, ex = bons.embed_bfp_rows(codes, sc)
        return mant[0].astype(np.float32) * np.float32(np.exp2(int(ex[0])))

    return TensorRef(mc, weights, gains, embed_row, kv_fp16=True)


def _oracle_hybrid(dec, mc, seed):
    """TensorRef over a hybrid's weights in HBM: ternary rows checked against the host hash, the
    Q8 beta/alpha rows and the DeltaNet float tensors read back (fp16(q * scale) as fastref caches
    Q8 weights)."""
    rng = np.random.default_rng(seed)
    E, hd, F, V = mc.n_embd, mc.head_dim, mc.ffn_dim, mc.vocab
    nq, nvh = mc.dn_num_k_heads * mc.dn_k_head_dim, mc.dn_num_v_heads * mc.dn_v_head_dim
    C_ = 2 * nq + nvh
    qrows = mc.n_head * hd * (2 if mc.attn_gated else 1)
    weights, gains, dn = {}, {}, {}
    for l in range(mc.n_layer):
        if mc.layer_type(l) == "deltanet":
            shapes = {L.ROLE_ATTN_QKV: (C_, E), L.ROLE_ATTN_ZGATE: (nvh, E), L.ROLE_SSM_OUT: (E, nvh)}
            for role in (L.ROLE_SSM_BETA, L.ROLE_SSM_ALPHA):
                raw = np.asarray(dec.read_tensor(role, l)).reshape(-1)
                rb = L.row_bytes(E, L.KIND_Q8)
                sc, q = bons.decode_rows(L.KIND_Q8, E, raw[:mc.dn_num_v_heads * rb].reshape(mc.dn_num_v_heads, rb))
                w = (q.astype(np.float16).reshape(q.shape[0], -1, 32) * sc[:, :, None]).astype(np.float16)
                weights[(role, l)] = w.reshape(q.shape[0], E).astype(np.float32)
            for role, n in ((L.ROLE_SSM_CONV, C_ * mc.dn_conv_kernel), (L.ROLE_SSM_A, mc.dn_num_v_heads),
                            (L.ROLE_SSM_DT, mc.dn_num_v_heads), (L.ROLE_SSM_NORM, mc.dn_v_head_dim)):
                dn[(role, l)] = dec.read_tensor(role, l).view(np.float32)[:n].copy()
            norm_roles = ((L.ROLE_ATTN_NORM, E), (L.ROLE_FFN_NORM, E))
        else:
            shapes = {L.ROLE_ATTN_Q: (qrows, E), L.ROLE_ATTN_K: (mc.n_kv_head * hd, E),
                      L.ROLE_ATTN_V: (mc.n_kv_head * hd, E), L.ROLE_ATTN_OUT: (E, mc.n_head * hd)}
            norm_roles = ((L.ROLE_ATTN_NORM, E), (L.ROLE_FFN_NORM, E), (L.ROLE_ATTN_Q_NORM, hd),
                          (L.ROLE_ATTN_K_NORM, hd))
        shapes.update({L.ROLE_FFN_GATE: (F, E), L.ROLE_FFN_UP: (F, E), L.ROLE_FFN_DOWN: (E, F)})
        for role, (r, c) in shapes.items():
            w, raw = _dequant(dec.read_tensor(role, l), r, c)
            _check_rows(raw, r, c, seed, role, l, rng)
            weights[(role, l)] = w
        for role, n in norm_roles:
            gains[(role, l)] = dec.read_tensor(role, l).view(np.float32)[:n].copy()
    gains[(L.ROLE_OUT_NORM, 0)] = dec.read_tensor(L.ROLE_OUT_NORM, 0).view(np.float32)[:E].copy()
    emb_raw = np.asarray(dec.read_tensor(L.ROLE_TOK_EMB, 0)).reshape(-1)
    rb = L.row_bytes(E, TRIT5)
    emb_raw = emb_raw[:V * rb].reshape(V, rb)
    _check_rows(emb_raw, V, E, seed, L.ROLE_TOK_EMB, 0, rng)
    w, raw = _dequant(dec.read_tensor(L.ROLE_LM_HEAD, 0), V, E)
    _check_rows(raw, V, E, seed, L.ROLE_LM_HEAD, 0, rng)
    weights[(L.ROLE_LM_HEAD, 0)] = w

    def embed_row(tok):
        sc, codes = bons.decode_rows(TRIT5, E, emb_raw[tok:tok + 1])
        mant, ex = bons.embed_bfp_rows(codes, sc)
        return mant[0].astype(np.float32) * np.float32(np.exp2(int(ex[0])))

    return TensorRef(mc, weights, gains, embed_row, kv_fp16=True, dn_tensors=dn)


@pytest.mark.timeout(1200)
def test_full_width_27b_hybrid_matches_the_oracle():
    """One Gated DeltaNet layer and one gated attention layer at the full Qwen3.5-27B width (5120
    wide; 48 v / 16 k DeltaNet heads of 128; 24 q / 4 kv heads of 256, 64 RoPE dims; FFN 17408)
    with the full 248320-row ternary head: the logits at the last 8 positions of a 64-token prompt
    (the DeltaNet state and conv window carried over 64 positions) within 2e-3 of the oracle, then
    16 greedy tokens identical to the oracle's; the batched prefill of the same prompt gives the
    same last-position logits within 2e-3."""
    from trixium_amd.model import Decoder
    mc = C.QWEN35_27B.replace(name="qwen3.5-27b-shape-2l", n_layer=2, layer_types=("deltanet", "attn"),
                              max_ctx=128)
    seed = 27
    dec = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=16)
    print("27b: reading the weights back", flush=True)
    ref = _oracle_hybrid(dec, mc, seed)
    prompt = synth.random_prompt(mc, 64, seed)
    errs, want = [], None
    for i, t in enumerate(prompt):
        got = dec.forward([t])
        want = ref.step(t, want_logits=i >= len(prompt) - 8)
        if want is not None:
            errs.append(_rel_err(got, want))
    print(f"27b: last 8 prompt positions max rel err {max(errs):.2e}", flush=True)
    assert max(errs) <= 2e-3
    ids, lg = [], want
    for i in range(16):
        ids.append(int(np.argmax(lg)))
        if i + 1 < 16:
            lg = ref.step(ids[-1])
    got = dec.generate_fresh(prompt, 16)
    assert got == ids
    dec.close()
    pre = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=16, prefill_chunk=32)
    assert _rel_err(pre.forward(prompt), want) <= 2e-3
    assert pre.generate_fresh(prompt, 16) == ids


@pytest.mark.timeout(900)
@pytest.mark.parametrize("shape", ["8b", "1.7b"])
def test_full_width_two_layers_match_the_oracle(shape):
    """Two layers at the full width with the full LM head: logits at all 32 prompt positions
    within 2e-3 of the oracle, then 64 greedy tokens identical to the oracle's."""
    from trixium_amd.model import Decoder
    base = C.QWEN3_8B if shape == "8b" else C.QWEN3_1P7B
    mc = base.replace(name=base.name + "-2l", n_layer=2, max_ctx=128)
    seed = 21 if shape == "8b" else 22
    dec = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=N_GREEDY)
    assert dec.packed_ops & 31 == 31          # every projection of a dense model on the packed GEMV
    print(f"{shape}: reading the weights back", flush=True)
    ref = _oracle(dec, mc, seed)
    prompt = synth.random_prompt(mc, N_PROMPT, seed)
    errs, want = [], None
    for t in prompt:
        got = dec.forward([t])
        want = ref.step(t)
        errs.append(_rel_err(got, want))
    print(f"{shape}: prompt positions max rel err {max(errs):.2e}", flush=True)
    assert max(errs) <= 2e-3
    ids = []
    lg = want
    for i in range(N_GREEDY):
        ids.append(int(np.argmax(lg)))
        if i + 1 < N_GREEDY:
            lg = ref.step(ids[-1])
    got = dec.generate_fresh(prompt, N_GREEDY)
    n_same = next((i for i, (a, b) in enumerate(zip(got, ids)) if a != b), N_GREEDY)
    print(f"{shape}: greedy tokens identical for {n_same} of {N_GREEDY}", flush=True)
    assert got == ids
    assert _rel_err(dec.logits(), lg) <= 2e-3


@pytest.mark.timeout(900)
@pytest.mark.parametrize("shape", ["8b", "1.7b"])
def test_full_depth_properties(shape):
    """Every layer at the headline shape (36 layers at 8B, 28 at 1.7B): graph replay of the
    position bitwise equal to eager launches; the packed GEMV against the row-packet GEMV within
    2e-3 at three positions (the row-packet path rounds its input to int16 per 128 group); finite
    logits."""
    from trixium_amd.model import Decoder
    mc = (C.QWEN3_8B if shape == "8b" else C.QWEN3_1P7B).replace(max_ctx=64)
    seed = 31
    prompt = synth.random_prompt(mc, 12, seed)
    a = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=16, use_graph=True)
    la = [a.forward(prompt)] + [a.forward([t]) for t in (5, 77777)]
    assert all(np.isfinite(v).all() for v in la)
    a.reset()
    ta = a.generate(prompt, 8)
    a.reset()
    lb = [a.forward(prompt, use_graph=False)] + [a.forward([t], use_graph=False) for t in (5, 77777)]
    for x, y in zip(la, lb):
        assert np.array_equal(x, y)
    a.reset()
    assert a.generate(prompt, 8, use_graph=False) == ta
    a.close()
    r = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=16, packed_ops=0)
    lr = [r.forward(prompt)] + [r.forward([t]) for t in (5, 77777)]
    errs = [_rel_err(x, y) for x, y in zip(la, lr)]
    print(f"{shape} full depth: packed vs row-packet rel err {errs}", flush=True)
    assert max(errs) <= 2e-3


@pytest.mark.timeout(900)
@pytest.mark.parametrize("shape,block", [("8b", 128), ("27b", 256)])
def test_rotated_full_width_handoffs_match_separate_launches(shape, block):
    """A PrismML-rotated model at the full width (two layers; the 27B shape one Gated DeltaNet and
    one gated attention layer): the packed GEMVs handing partial sums on, each rotating its input
    in the prologue (blocks inside the K-slice), against every projection on the row-packet kernel
    after a separate rotation launch (the path without handoffs): logits at 8 positions within
    2e-3 (the row-packet kernel rounds its input to int16 per 128-group) and the same greedy
    tokens."""
    from trixium_amd.model import Decoder
    if shape == "8b":
        mc = C.QWEN3_8B.replace(name="qwen3-8b-shape-2l", n_layer=2, max_ctx=64)
    else:
        mc = C.QWEN35_27B.replace(name="qwen3.5-27b-shape-2l", n_layer=2, layer_types=("deltanet", "attn"),
                                  max_ctx=64)
    seed = 51
    prompt = synth.random_prompt(mc, 8, seed)
    a = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=8, hadamard_block=block)
    b = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=8, hadamard_block=block, packed_ops=0)
    la = [a.forward(prompt[:4])] + [a.forward([t]) for t in prompt[4:]]
    lb = [b.forward(prompt[:4])] + [b.forward([t]) for t in prompt[4:]]
    errs = [_rel_err(x, y) for x, y in zip(la, lb)]
    print(f"{shape} rotated ({block}): handoffs vs separate launches rel err {max(errs):.2e}", flush=True)
    assert max(errs) <= 2e-3
    assert a.generate_fresh(prompt, 8) == b.generate_fresh(prompt, 8)
    a.close()
    b.close()
