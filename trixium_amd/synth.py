"""Synthetic random-ternary models.

Small models are drawn with numpy's default_rng in a fixed call order (the pattern of the
reference's tinygen, model/tinygen.py:39-84) with the measured distributions: trits with
P(0) = 0.4 and P(-1) = P(+1) = 0.3, fp16 group scales U(0.01, 0.05), RMSNorm gains U(0.8, 1.2),
fp16 embeddings N(0, 0.02).

Large models are never materialised on the host: their weights come from a counter-based hash
(splitmix64 of (seed, tensor id, element)), which the device generator (csrc/trx_ops.hip:
synth_ternary_kernel, synth_f32_kernel) evaluates in place in HBM and `hashed_codes` /
`hashed_scales` / `hashed_uniform` below evaluate for any rows on the host, so a CPU check can
rebuild exactly the rows it needs.
"""

import numpy as np

from . import layout as L
from .bons import TensorSpec, write_image

P_NEG, P_ZERO = 0.3, 0.4          # P(code 0) = P(w = -1), P(code 1) = P(w = 0)
SCALE_LO, SCALE_HI = 0.01, 0.05


def _ternary(rng, name, role, layer, rows, cols):
    u = rng.random((rows, cols))
    codes = np.where(u < P_NEG, 0, np.where(u < P_NEG + P_ZERO, 1, 2)).astype(np.uint8)
    scales = rng.uniform(SCALE_LO, SCALE_HI, (rows, cols // L.GROUP)).astype(np.float16)
    return TensorSpec(name, role, layer, L.KIND_TERNARY, rows, cols, scales=scales, values=codes)


def _q8(rng, name, role, layer, rows, cols):
    scales = rng.uniform(0.005, 0.02, (rows, cols // L.GROUP_Q8)).astype(np.float16)
    values = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    return TensorSpec(name, role, layer, L.KIND_Q8, rows, cols, scales=scales, values=values)


def _norm(rng, name, role, layer, cols):
    v = rng.uniform(0.8, 1.2, (1, cols)).astype(np.float32)
    return TensorSpec(name, role, layer, L.KIND_F32, 1, cols, values=v, flags=L.FLAG_REPLICATED)


def _f32(name, role, layer, values):
    return TensorSpec(name, role, layer, L.KIND_F32, values.shape[0], values.shape[1],
                      values=values.astype(np.float32), flags=L.FLAG_REPLICATED)


def small_model_tensors(cfg, seed=0, fp16_embedding=True):
    """Tensor list of a small random model. fp16_embedding: the token embedding is fp16
    N(0, 0.02), stored as the int16 lookup table plus (tied) an F32 LM head holding the same
    fp16-exact values; otherwise it is a ternary token_embd (tied head) or a separate ternary
    output.weight (untied)."""
    rng = np.random.default_rng(seed)
    t = []
    emb = None
    if fp16_embedding:
        emb = rng.normal(0.0, 0.02, (cfg.vocab, cfg.n_embd)).astype(np.float16)
    else:
        t.append(_ternary(rng, "token_embd.weight", L.ROLE_TOK_EMB, 0, cfg.vocab, cfg.n_embd))
    nk, hk, nv, hv = cfg.dn_num_k_heads, cfg.dn_k_head_dim, cfg.dn_num_v_heads, cfg.dn_v_head_dim
    for l in range(cfg.n_layer):
        p = f"blk.{l}."
        t.append(_norm(rng, p + "attn_norm.weight", L.ROLE_ATTN_NORM, l, cfg.n_embd))
        if cfg.layer_type(l) == "deltanet":
            C = 2 * nk * hk + nv * hv
            t.append(_ternary(rng, p + "attn_qkv.weight", L.ROLE_ATTN_QKV, l, C, cfg.n_embd))
            t.append(_ternary(rng, p + "attn_gate.weight", L.ROLE_ATTN_ZGATE, l, nv * hv, cfg.n_embd))
            t.append(_q8(rng, p + "ssm_beta.weight", L.ROLE_SSM_BETA, l, nv, cfg.n_embd))
            t.append(_q8(rng, p + "ssm_alpha.weight", L.ROLE_SSM_ALPHA, l, nv, cfg.n_embd))
            taps = rng.uniform(-0.5, 0.5, (C, cfg.dn_conv_kernel)).astype(np.float32)
            t.append(_f32(p + "ssm_conv1d.weight", L.ROLE_SSM_CONV, l, taps))
            t.append(_f32(p + "ssm_a", L.ROLE_SSM_A, l, -np.exp(rng.uniform(-1.5, 0.5, (1, nv)))))
            t.append(_f32(p + "ssm_dt.bias", L.ROLE_SSM_DT, l, rng.uniform(-2.0, 0.5, (1, nv))))
            t.append(_norm(rng, p + "ssm_norm.weight", L.ROLE_SSM_NORM, l, hv))
            t.append(_ternary(rng, p + "ssm_out.weight", L.ROLE_SSM_OUT, l, cfg.n_embd, nv * hv))
        else:
            qrows = 2 * cfg.q_dim if cfg.attn_gated else cfg.q_dim
            t.append(_ternary(rng, p + "attn_q.weight", L.ROLE_ATTN_Q, l, qrows, cfg.n_embd))
            t.append(_ternary(rng, p + "attn_k.weight", L.ROLE_ATTN_K, l, cfg.kv_dim, cfg.n_embd))
            t.append(_ternary(rng, p + "attn_v.weight", L.ROLE_ATTN_V, l, cfg.kv_dim, cfg.n_embd))
            t.append(_norm(rng, p + "attn_q_norm.weight", L.ROLE_ATTN_Q_NORM, l, cfg.head_dim))
            t.append(_norm(rng, p + "attn_k_norm.weight", L.ROLE_ATTN_K_NORM, l, cfg.head_dim))
            t.append(_ternary(rng, p + "attn_output.weight", L.ROLE_ATTN_OUT, l, cfg.n_embd, cfg.q_dim))
        t.append(_norm(rng, p + "ffn_norm.weight", L.ROLE_FFN_NORM, l, cfg.n_embd))
        t.append(_ternary(rng, p + "ffn_gate.weight", L.ROLE_FFN_GATE, l, cfg.ffn_dim, cfg.n_embd))
        t.append(_ternary(rng, p + "ffn_up.weight", L.ROLE_FFN_UP, l, cfg.ffn_dim, cfg.n_embd))
        t.append(_ternary(rng, p + "ffn_down.weight", L.ROLE_FFN_DOWN, l, cfg.n_embd, cfg.ffn_dim))
    t.append(_norm(rng, "output_norm.weight", L.ROLE_OUT_NORM, 0, cfg.n_embd))
    if emb is not None:
        from .bons import float_bfp_rows, emb16_specs
        t.extend(emb16_specs(*float_bfp_rows(emb.astype(np.float32))))
        t.append(TensorSpec("output.weight", L.ROLE_LM_HEAD, 0, L.KIND_F32, cfg.vocab, cfg.n_embd,
                            values=emb.astype(np.float32)))
    elif not cfg.tie_embeddings:
        t.append(_ternary(rng, "output.weight", L.ROLE_LM_HEAD, 0, cfg.vocab, cfg.n_embd))
    return t


def write_small_model(path, cfg, seed=0, trit5=True, fp16_embedding=True):
    tensors = small_model_tensors(cfg, seed, fp16_embedding)
    return write_image(cfg, tensors, 1, path, trit5=trit5)


def random_prompt(cfg, n=16, seed=0):
    return [int(t) for t in np.random.default_rng(seed).integers(0, cfg.vocab, n)]


# Counter-based generator (host side of the device generator in csrc/trx_ops.hip) ---------------------------------------

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(z):
    """splitmix64 finaliser over a uint64 array (wrapping arithmetic)."""
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def _key(seed, tensor_id, stream):
    return splitmix64(np.uint64((seed & 0xFFFFFFFF) << 32 | (tensor_id & 0xFFFFFF) << 8 | stream))


# Thresholds on a 16-bit uniform: code 0 below T0, code 1 below T1, else code 2.
CODE_T0 = 19661          # round(0.3 * 65536)
CODE_T1 = 45875          # round(0.7 * 65536)


def hashed_codes(seed, tensor_id, rows, cols):
    """Codes {0,1,2} of rows `rows` (array) of a (.., cols) hashed tensor: one 64-bit hash per
    4 consecutive columns, 16 bits per code."""
    rows = np.asarray(rows, dtype=np.uint64)
    key = _key(seed, tensor_id, 1)
    q = cols // 4
    ctr = rows[:, None] * np.uint64(q) + np.arange(q, dtype=np.uint64)[None, :]
    with np.errstate(over="ignore"):
        h = splitmix64(ctr ^ key)
    u = np.stack([(h >> np.uint64(16 * k)) & np.uint64(0xFFFF) for k in range(4)], axis=-1)
    u = u.reshape(len(rows), cols).astype(np.int64)
    return np.where(u < CODE_T0, 0, np.where(u < CODE_T1, 1, 2)).astype(np.uint8)


def hashed_uniform(seed, tensor_id, stream, idx, lo, hi):
    """float32 U(lo, hi) from the top 24 bits of the hash of each index."""
    key = _key(seed, tensor_id, stream)
    with np.errstate(over="ignore"):
        h = splitmix64(np.asarray(idx, dtype=np.uint64) ^ key)
    u = (h >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))
    return (np.float32(lo) + np.float32(hi - lo) * u.astype(np.float32)).astype(np.float32)


def hashed_scales(seed, tensor_id, rows, cols):
    rows = np.asarray(rows, dtype=np.int64)
    G = cols // L.GROUP
    idx = rows[:, None] * G + np.arange(G)[None, :]
    return hashed_uniform(seed, tensor_id, 2, idx, SCALE_LO, SCALE_HI).astype(np.float16)


GAIN_LO, GAIN_HI = 0.8, 1.2


def tensor_id(role, layer):
    return layer * 32 + role


def hashed_ternary(seed, role, layer, rows, cols, name):
    tid = tensor_id(role, layer)
    r = np.arange(rows)
    return TensorSpec(name, role, layer, L.KIND_TERNARY, rows, cols,
                      scales=hashed_scales(seed, tid, r, cols), values=hashed_codes(seed, tid, r, cols))


def hashed_gain(seed, role, layer, cols, name):
    v = hashed_uniform(seed, tensor_id(role, layer), 3, np.arange(cols), GAIN_LO, GAIN_HI)
    return TensorSpec(name, role, layer, L.KIND_F32, 1, cols, values=v.reshape(1, cols),
                      flags=L.FLAG_REPLICATED)


def hashed_model_tensors(cfg, seed=0):
    """The tensor list of a full-attention model with every value from the counter-based hash,
    as the device generator fills it: ternary token_embd, untied ternary output.weight unless
    cfg.tie_embeddings, RMSNorm gains U(0.8, 1.2). For small configs (CPU checks)."""
    if cfg.n_dn_layers:
        raise NotImplementedError("hashed DeltaNet tensors are not generated")
    E = cfg.n_embd
    t = [hashed_ternary(seed, L.ROLE_TOK_EMB, 0, cfg.vocab, E, "token_embd.weight")]
    for l in range(cfg.n_layer):
        p = f"blk.{l}."
        t.append(hashed_gain(seed, L.ROLE_ATTN_NORM, l, E, p + "attn_norm.weight"))
        t.append(hashed_ternary(seed, L.ROLE_ATTN_Q, l, cfg.q_dim, E, p + "attn_q.weight"))
        t.append(hashed_ternary(seed, L.ROLE_ATTN_K, l, cfg.kv_dim, E, p + "attn_k.weight"))
        t.append(hashed_ternary(seed, L.ROLE_ATTN_V, l, cfg.kv_dim, E, p + "attn_v.weight"))
        t.append(hashed_gain(seed, L.ROLE_ATTN_Q_NORM, l, cfg.head_dim, p + "attn_q_norm.weight"))
        t.append(hashed_gain(seed, L.ROLE_ATTN_K_NORM, l, cfg.head_dim, p + "attn_k_norm.weight"))
        t.append(hashed_ternary(seed, L.ROLE_ATTN_OUT, l, E, cfg.q_dim, p + "attn_output.weight"))
        t.append(hashed_gain(seed, L.ROLE_FFN_NORM, l, E, p + "ffn_norm.weight"))
        t.append(hashed_ternary(seed, L.ROLE_FFN_GATE, l, cfg.ffn_dim, E, p + "ffn_gate.weight"))
        t.append(hashed_ternary(seed, L.ROLE_FFN_UP, l, cfg.ffn_dim, E, p + "ffn_up.weight"))
        t.append(hashed_ternary(seed, L.ROLE_FFN_DOWN, l, E, cfg.ffn_dim, p + "ffn_down.weight"))
    t.append(hashed_gain(seed, L.ROLE_OUT_NORM, 0, E, "output_norm.weight"))
    if not cfg.tie_embeddings:
        t.append(hashed_ternary(seed, L.ROLE_LM_HEAD, 0, cfg.vocab, E, "output.weight"))
    return t
