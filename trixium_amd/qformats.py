"""GGUF block formats of the Bonsai models (numpy): the codecs the GGUF -> BONS converter reads.

Follows model/qformats.py (the PrismML llama.cpp fork's ggml-quants.c semantics):
- PQ2_0 (type 142) and the legacy g128 Q2_0 (type 42): 128 weights per 34-byte block, an fp16
  scale d then 32 bytes of 2-bit codes (weight j in byte j/4 at bit 2(j%4)); w = (q - 1) d.
  Type 42 is also upstream's group-64 Q2_0 (18 bytes per 64 weights); the payload size tells
  them apart (`q2_0_group`, model/qformats.py:84-95).
- PTQ1_0 (type 143): the same ternary codes five trits per byte, 28 bytes per 128 weights: 24
  bytes of five trits, 2 bytes of four trits, the fp16 scale (model/qformats.py:102-178).
- Q1_0 (type 41): 18 bytes per 128 weights, bit set -> +d, clear -> -d (model/qformats.py:180-224).
- Q8_0 (type 8): 34 bytes per 32 weights, fp16 d then int8 q; w = q d (model/qformats.py:226-257).
- F32 (0), F16 (1) and BF16 (30) payloads.
"""

import numpy as np

GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
GGML_Q1_0 = 41       # PrismML fork, 1-bit g128
GGML_Q2_0 = 42       # PrismML fork's g128 2-bit block in older files; upstream's g64 block now
GGML_PQ2_0 = 142     # PrismML fork, the g128 2-bit block under its current id
GGML_PTQ1_0 = 143    # PrismML fork, g128 trits five per byte

QK_Q2_0, BLOCK_Q2_0 = 128, 34
QK_PTQ1_0, BLOCK_PTQ1_0 = 128, 28
QK_Q1_0, BLOCK_Q1_0 = 128, 18
QK_Q8_0, BLOCK_Q8_0 = 32, 34


def _u8(raw):
    return raw if isinstance(raw, np.ndarray) and raw.dtype == np.uint8 else np.frombuffer(raw, np.uint8)


def _blocks(raw, block, what):
    raw = _u8(raw)
    if raw.size % block:
        raise ValueError(f"{what} payload of {raw.size} bytes is not a multiple of {block}")
    return raw.reshape(-1, block)


def _scales(blocks, at):
    return np.ascontiguousarray(blocks[:, at:at + 2]).view(np.float16).reshape(-1)


def _put_scales(out, at, scales):
    out[:, at:at + 2] = np.asarray(scales, np.float16).reshape(-1, 1).view(np.uint8)


# 2-bit (PQ2_0 / g128 Q2_0) -----------------------------------------------------------------------

def q2_0_unpack(raw):
    """(scales fp16 (nb,), codes uint8 (nb, 128) in 0..3)."""
    b = _blocks(raw, BLOCK_Q2_0, "Q2_0")
    shifts = np.array([0, 2, 4, 6], np.uint8)
    codes = (b[:, 2:, None] >> shifts) & 3                      # (nb, 32, 4): byte, position
    return _scales(b, 0), codes.reshape(-1, QK_Q2_0).astype(np.uint8)


def q2_0_scales(raw):
    return _scales(_blocks(raw, BLOCK_Q2_0, "Q2_0"), 0)


def q2_0_pack(scales, codes):
    codes = np.asarray(codes, np.uint8)
    if codes.ndim != 2 or codes.shape[1] != QK_Q2_0 or codes.max(initial=0) > 3:
        raise ValueError("codes must be (nb, 128) in 0..3")
    nb = codes.shape[0]
    q = codes.reshape(nb, 32, 4).astype(np.uint8)
    out = np.empty((nb, BLOCK_Q2_0), np.uint8)
    _put_scales(out, 0, scales)
    out[:, 2:] = q[:, :, 0] | (q[:, :, 1] << 2) | (q[:, :, 2] << 4) | (q[:, :, 3] << 6)
    return out.reshape(-1)


def q2_0_group(raw, n_elements):
    """128 when a type-42 payload holds the g128 block (34 B per 128), 64 for upstream's g64 block
    (18 B per 64); ValueError otherwise."""
    n = raw.size if isinstance(raw, np.ndarray) else len(raw)
    if n * QK_Q2_0 == n_elements * BLOCK_Q2_0:
        return 128
    if n * 64 == n_elements * 18:
        return 64
    raise ValueError(f"Q2_0 payload of {n} bytes fits neither g128 nor g64 for {n_elements} weights")


def q2_0_dequant(raw):
    s, c = q2_0_unpack(raw)
    return ((c.astype(np.float32) - 1.0) * s.astype(np.float32)[:, None]).reshape(-1)


# Dense trits (PTQ1_0) ------------------------------------------------------------------------------

def _ptq1_order():
    """Weight index of (byte, trit) in a PTQ1_0 block. The 24 five-trit bytes come in runs (16
    bytes, then 8: the widest run of 32, 16 or 8 that still fits); run bytes j..j+c-1 hold weights
    base + n c + m for trit n of byte j + m. The two four-trit bytes hold weights 120 + 2 n + h."""
    qs = np.zeros((24, 5), np.int64)
    e, j = 0, 0
    for c in (32, 16, 8):
        while j + c <= 24:
            qs[j:j + c, :] = e + np.arange(5)[None, :] * c + np.arange(c)[:, None]
            e += 5 * c
            j += c
    qh = 120 + 2 * np.arange(4)[None, :] + np.arange(2)[:, None]   # (2 bytes, 4 trits)
    return qs, qh


_QS_IDX, _QH_IDX = _ptq1_order()


def _ptq1_runs():
    """(first byte, bytes, first weight) of each run of five-trit bytes: within a run, trit n of
    byte j + m is weight base + n c + m, i.e. the run's weights are its bytes' trits digit-major."""
    runs, e, j = [], 0, 0
    for c in (32, 16, 8):
        while j + c <= 24:
            runs.append((j, c, e))
            e += 5 * c
            j += c
    return runs


_RUNS = _ptq1_runs()
_POW3 = np.array([1, 3, 9, 27, 81], np.uint16)


def _trits(q, n):
    """The first n base-3 digits of fixed-point bytes q, (nb, bytes, n): digit k = ((q 3^k) mod
    256) 3 >> 8, computed in uint8 (the multiply wraps mod 256; t 3 >> 8 is (t >= 86) + (t >= 171))."""
    q = np.asarray(q, np.uint8)
    out = np.empty(q.shape + (n,), np.uint8)
    for k in range(n):
        t = q * np.uint8(3 ** k)
        out[..., k] = (t >= 86).view(np.uint8) + (t >= 171).view(np.uint8)
    return out


def ptq1_0_unpack(raw):
    """(scales fp16 (nb,), codes uint8 (nb, 128) in 0..2)."""
    b = _blocks(raw, BLOCK_PTQ1_0, "PTQ1_0")
    nb = b.shape[0]
    codes = np.empty((nb, QK_PTQ1_0), np.uint8)
    for j, c, e in _RUNS:
        codes[:, e:e + 5 * c] = _trits(b[:, j:j + c], 5).transpose(0, 2, 1).reshape(nb, 5 * c)
    codes[:, 120:128] = _trits(b[:, 24:26], 4).transpose(0, 2, 1).reshape(nb, 8)   # weight 120 + 2n + h
    return _scales(b, 26), codes


def ptq1_0_scales(raw):
    return _scales(_blocks(raw, BLOCK_PTQ1_0, "PTQ1_0"), 26)


def _fixed_point(v):
    """A base-3 number of five digits (< 243) as the byte ceil(v 256 / 243): multiplying by 3^k
    mod 256 and taking the top two bits then yields digit k, most significant first."""
    return ((v.astype(np.uint32) * 256 + 242) // 243).astype(np.uint8)


def ptq1_0_pack(scales, codes):
    codes = np.asarray(codes, np.uint8)
    if codes.ndim != 2 or codes.shape[1] != QK_PTQ1_0 or codes.max(initial=0) > 2:
        raise ValueError("codes must be (nb, 128) in 0..2")
    nb = codes.shape[0]
    w5 = np.array([81, 27, 9, 3, 1], np.uint32)               # digit 0 most significant
    qs = (codes[:, _QS_IDX].astype(np.uint32) * w5).sum(axis=2)
    qh = (codes[:, _QH_IDX].astype(np.uint32) * w5[:4]).sum(axis=2)   # four digits, top aligned
    out = np.empty((nb, BLOCK_PTQ1_0), np.uint8)
    out[:, :24] = _fixed_point(qs)
    out[:, 24:26] = _fixed_point(qh)
    _put_scales(out, 26, scales)
    return out.reshape(-1)


def ptq1_0_dequant(raw):
    s, c = ptq1_0_unpack(raw)
    return ((c.astype(np.float32) - 1.0) * s.astype(np.float32)[:, None]).reshape(-1)


# 1-bit (Q1_0) --------------------------------------------------------------------------------------

def q1_0_unpack(raw):
    """(scales fp16 (nb,), bits uint8 (nb, 128)); weight j is bit j%8 of byte j/8."""
    b = _blocks(raw, BLOCK_Q1_0, "Q1_0")
    return _scales(b, 0), np.unpackbits(b[:, 2:], axis=1, bitorder="little")


def q1_0_pack(scales, bits):
    bits = np.asarray(bits, np.uint8)
    if bits.ndim != 2 or bits.shape[1] != QK_Q1_0:
        raise ValueError("bits must be (nb, 128)")
    out = np.empty((bits.shape[0], BLOCK_Q1_0), np.uint8)
    _put_scales(out, 0, scales)
    out[:, 2:] = np.packbits(bits, axis=1, bitorder="little")
    return out.reshape(-1)


def q1_0_dequant(raw):
    s, bits = q1_0_unpack(raw)
    return ((bits.astype(np.float32) * 2.0 - 1.0) * s.astype(np.float32)[:, None]).reshape(-1)


def q1_0_to_ternary_codes(raw):
    """1-bit weights as ternary codes for the ternary GEMV: -1 -> code 0, +1 -> code 2."""
    s, bits = q1_0_unpack(raw)
    return s, (bits * 2).astype(np.uint8)


# Q8_0 ------------------------------------------------------------------------------------------------

def q8_0_unpack(raw):
    b = _blocks(raw, BLOCK_Q8_0, "Q8_0")
    return _scales(b, 0), np.ascontiguousarray(b[:, 2:]).view(np.int8)


def q8_0_pack(scales, quants):
    quants = np.asarray(quants, np.int8)
    if quants.ndim != 2 or quants.shape[1] != QK_Q8_0:
        raise ValueError("quants must be (nb, 32)")
    out = np.empty((quants.shape[0], BLOCK_Q8_0), np.uint8)
    _put_scales(out, 0, scales)
    out[:, 2:] = quants.view(np.uint8)
    return out.reshape(-1)


def q8_0_dequant(raw):
    s, q = q8_0_unpack(raw)
    return (q.astype(np.float32) * s.astype(np.float32)[:, None]).reshape(-1)


def q8_0_quant(w):
    """Absmax-per-32 quantisation to Q8_0 bytes (d = amax/127, q = round(w/d))."""
    g = np.asarray(w, np.float32).reshape(-1, QK_Q8_0)
    d = np.abs(g).max(axis=1) / 127.0
    inv = np.divide(1.0, d, out=np.zeros_like(d), where=d > 0)
    q = np.clip(np.rint(g * inv[:, None]), -127, 127).astype(np.int8)
    return q8_0_pack(d.astype(np.float16), q)


# Float payloads ------------------------------------------------------------------------------------

def f32_dequant(raw):
    return np.frombuffer(np.ascontiguousarray(_u8(raw)).tobytes(), np.float32).copy()


def f16_dequant(raw):
    return np.frombuffer(np.ascontiguousarray(_u8(raw)).tobytes(), np.float16).astype(np.float32)


def bf16_dequant(raw):
    """bfloat16: the top half of an fp32."""
    h = np.frombuffer(np.ascontiguousarray(_u8(raw)).tobytes(), np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


DEQUANT = {
    GGML_F32: f32_dequant,
    GGML_F16: f16_dequant,
    GGML_Q8_0: q8_0_dequant,
    GGML_BF16: bf16_dequant,
    GGML_Q1_0: q1_0_dequant,
    GGML_Q2_0: q2_0_dequant,      # the g128 block only (check q2_0_group first)
    GGML_PQ2_0: q2_0_dequant,
    GGML_PTQ1_0: ptq1_0_dequant,
}
