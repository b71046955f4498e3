"""Integer engine contract, restated in numpy (test infrastructure only, see oracle/__init__.py).

Restates model/bitexact.py:35-144 and the activation quantizer of model/mirror.py:39-51:

    gs[m, g]  = sum over the group's 128 lanes of (code - 1) * x8          exact, |gs| <= 16256
    fp16 s    = m11 * 2**e16                                                exact split
    acc[m]    = sum_g  (gs * m11) << (e16 + B)   (arithmetic >> for a negative shift)
    y[m]      = acc >> R                                                    int32
"""

import numpy as np

ACC_BITS = 48
RESULT_BITS = 32
GS_MAX = 128 * 127
GS_MAX_Q8 = 32 * 127 * 127


def rne_shift(v, k):
    """Round-half-even right shift (model/bitexact.py:35-46)."""
    v = np.asarray(v, dtype=np.int64)
    if k == 0:
        return v.copy()
    q = v >> k
    half_bit = (v >> (k - 1)) & 1
    rest = (v & ((1 << (k - 1)) - 1)) != 0
    return q + (half_bit & (rest | ((q & 1) == 1))).astype(np.int64)


def fp16_decompose(s):
    """fp16 -> (m11, e16) with s == m11 * 2**e16 (model/bitexact.py:56-70)."""
    bits = np.asarray(s, dtype=np.float16).view(np.uint16).astype(np.int64)
    E = (bits >> 10) & 0x1F
    assert not np.any(E == 0x1F), "fp16 inf/nan in scales"
    frac = bits & 0x3FF
    sign = np.where(bits & 0x8000, -1, 1)
    m11 = np.where(E > 0, frac + 1024, frac) * sign
    e16 = np.where(E > 0, E - 25, -24)
    return m11, e16


def choose_scale_bias(e16_all, target_top=12):
    """B = 12 - max(e16) (model/bitexact.py:78-81)."""
    return int(target_top - np.max(e16_all))


def tensor_acc_bound(scales_f16, B, gs_max=GS_MAX):
    """Worst |acc| over the tensor's rows (model/bitexact.py:83-90)."""
    m11, e16 = fp16_decompose(scales_f16)
    per = np.abs(m11).astype(np.float64) * gs_max * np.exp2((e16 + B).astype(np.float64))
    return np.ceil(per).sum(axis=1).max()


def choose_result_shift(scales_f16, B, gs_max=GS_MAX):
    """Smallest R with bound >> R inside int32 (model/bitexact.py:92-97)."""
    bound = tensor_acc_bound(scales_f16, B, gs_max)
    R = 0
    while bound / (1 << R) >= 2**(RESULT_BITS - 1):
        R += 1
    return R


def group_sums(codes, x8, group=128, offset=1):
    """Exact per-group sums of (code - offset) * x (int64 (M, G))."""
    M, K = codes.shape
    w = codes.astype(np.int64) - offset
    return (w * np.asarray(x8, dtype=np.int64)[None, :]).reshape(M, K // group, group).sum(axis=2)


def _shift_accumulate(gs, scales_f16, B, R):
    m11, e16 = fp16_decompose(scales_f16)
    prod = gs * m11
    sh = e16 + B
    contrib = np.where(sh >= 0, prod << np.maximum(sh, 0), prod >> np.maximum(-sh, 0))
    acc = contrib.sum(axis=1)
    assert np.all(np.abs(acc) < 2**(ACC_BITS - 1)), "int48 accumulator overflow"
    res = acc >> R
    assert np.all(np.abs(res) < 2**(RESULT_BITS - 1)), "int32 result overflow"
    return res.astype(np.int32), acc


def matvec_ternary(scales_f16, codes, x8, B, R):
    """Exact engine matvec (model/bitexact.py:101-119): scales (M, G) fp16, codes (M, K) in
    {0,1,2}, x8 (K,) int8 -> int32 (M,)."""
    return _shift_accumulate(group_sums(codes, x8), scales_f16, B, R)[0]


def matvec_ternary_rows(scales_f16, codes, x8_rows, B, R):
    """Multi-row engine matvec (model/bitexact.py:121-125): every row of x8_rows (n, K) is the
    single-row matvec of that row -> int32 (n, M)."""
    return np.stack([matvec_ternary(scales_f16, codes, x8, B, R) for x8 in x8_rows])


def matvec_q8(scales_f16, q8w, x8, B, R):
    """Q8 row-dot mode (model/bitexact.py:127-144): group 32, w = q8 * scale."""
    return _shift_accumulate(group_sums(q8w, x8, group=32, offset=0), scales_f16, B, R)[0]


def lroundf(x):
    """C lroundf: half away from zero."""
    x = np.asarray(x)
    return np.where(x >= 0, np.floor(x + 0.5), np.ceil(x - 0.5)).astype(np.int64)


def quantize_f_pow2(x):
    """fp32 activations -> (int8, e8): e8 = frexp(amax) - 7, x8 = clip(lroundf(x * 2**-e8), +-127)
    (model/mirror.py:45-51, firmware/infer.c:144)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max() if x.size else 0.0
    if amax == 0:
        return np.zeros(len(x), dtype=np.int8), 0
    e8 = int(np.frexp(np.float32(amax))[1]) - 7
    q = lroundf(x * np.float32(np.exp2(-e8)))
    return np.clip(q, -127, 127).astype(np.int8), e8


def restored_row_exact(scales_f16, codes, signs, hblock):
    """A rotated embedding row restored to the plain basis in integers (model/bons.py:262-295,
    the firmware's embed_row_restore for images without the int16 table):
      v = (code - 1) * m11 aligned to the row's smallest fp16 exponent (int64);
      y = s * (H v) per block of hblock columns (natural-order Walsh-Hadamard butterflies);
      the absmax mantissa normalised into [2^14, 2^15) by a round-half-to-even right shift (or a
      left shift), clipped to +-32767; exponent = e16min - floor(log2(hblock) / 2) + shift.
    -> (int16 row, int exponent)."""
    m11, e16 = fp16_decompose(np.asarray(scales_f16).reshape(-1))
    e16min = int(e16.min())
    q = np.asarray(codes).astype(np.int64).reshape(len(m11), -1) - 1
    v = (q * (m11.astype(np.int64) << (e16 - e16min).astype(np.int64))[:, None]).reshape(-1)
    n = v.size
    h = 1
    while h < hblock:
        v = v.reshape(n // (2 * h), 2, h)
        v = np.stack([v[:, 0] + v[:, 1], v[:, 0] - v[:, 1]], axis=1).reshape(-1)
        h *= 2
    y = v * np.asarray(signs).astype(np.int64)
    fexp = -((int(hblock).bit_length() - 1) // 2)
    amax = int(np.abs(y).max())
    if amax == 0:
        return np.zeros(n, dtype=np.int16), 0
    r = amax.bit_length() - 15
    if r > 0:
        mant = np.where(y < 0, -rne_shift(np.abs(y), r), rne_shift(np.abs(y), r))
    else:
        mant = y << -r
    return np.clip(mant, -32767, 32767).astype(np.int16), e16min + fexp + r
