"""Host-side fixed-point helpers of the engine contract: the exact fp16 split of a group scale and
the per-tensor scale bias B / result shift R an image stores with every quantized tensor
(the rules of model/bitexact.py:56-97, restated).

    fp16 s = m11 * 2**e16 exactly (m11 signed 11-bit, e16 = E - 25, or -24 for subnormals)
    B = 12 - max(e16)                     largest scale's product lands at bit 12
    R = smallest shift with (worst-case |acc|) >> R < 2**31
"""

import numpy as np

GS_MAX = 128 * 127            # |group sum| bound, ternary (128 lanes x |x8| <= 127)
GS_MAX_Q8 = 32 * 127 * 127    # Q8 row-dot bound


def fp16_split(s):
    """fp16 array -> (m11 int64, e16 int64) with s == m11 * 2**e16 exactly."""
    bits = np.asarray(s, dtype=np.float16).view(np.uint16).astype(np.int64)
    expo = (bits >> 10) & 0x1F
    if np.any(expo == 0x1F):
        raise ValueError("inf/nan fp16 scale")
    frac = bits & 0x3FF
    mag = np.where(expo > 0, frac | 0x400, frac)
    m11 = np.where(bits & 0x8000, -mag, mag)
    e16 = np.where(expo > 0, expo - 25, -24)
    return m11, e16


def scale_bias(scales):
    _, e16 = fp16_split(scales)
    return int(12 - e16.max())


def result_shift(scales, bias, gs_max=GS_MAX):
    """Smallest R keeping the worst-case accumulator of any row inside int32 after >> R."""
    m11, e16 = fp16_split(scales)
    mag = np.abs(m11).astype(np.float64) * gs_max * np.exp2((e16 + bias).astype(np.float64))
    bound = np.ceil(mag).sum(axis=1).max()
    r = 0
    while bound / (1 << r) >= 2.0**31:
        r += 1
    return r
