"""PrismML's rotated weight basis (the Bonsai hybrids): host-side pieces.

A folded weight W' = W R diag(s) is applied as y = W' (R (s x)) blockwise on the input, with R
the natural-order Sylvester Walsh-Hadamard matrix of the block, R[i][j] = (-1)^popcount(i & j) /
sqrt(block) (symmetric, its own inverse), s a +-1 sign per input column. A folded embedding table
holds z = R diag(s) e and is restored as e = s (R z) after the lookup (model/golden.py:250-289).

In a BONS image the rotation of each input width is a set of ternary block tensors (role
hadamard, layer = width index * 256 + block): rows R_pm1[i] * s, scale a power of two (1/sqrt(block)
for an even power of two; 2^-floor(log2(block) / 2) for an odd one, the remaining 2^-0.5 folded
into every rotated weight's scales by the converter), model/convert.py:84-106.
"""

import numpy as np

from . import layout as L


def sign_matrix(block):
    """The +-1 Sylvester matrix, float32: (-1)^popcount(i & j)."""
    i = np.arange(block)
    par = i[:, None] & i[None, :]
    odd = np.zeros_like(par)
    while par.any():
        odd ^= par & 1
        par >>= 1
    return np.where(odd & 1, -1.0, 1.0).astype(np.float32)


def matrix(block):
    """R, normalized: sign_matrix / sqrt(block), float32."""
    return sign_matrix(block) / np.sqrt(float(block))


def image_scales(block):
    """(rotation tensor scale, weight fold) of an image's rotation: a power of two either way."""
    k = int(block).bit_length() - 1
    if block != 1 << k:
        raise ValueError(f"Hadamard block {block} is not a power of two")
    return 2.0 ** -(k // 2), (1.0 if k % 2 == 0 else 2.0 ** -0.5)


def image_gain(block):
    """What the rotation tensors (and the restored table) carry over the normalized transform:
    sqrt(2) for an odd power-of-two block, 1 otherwise."""
    return image_scales(block)[0] * np.sqrt(float(block))


def restore(z, signs, block):
    """e = s (R z) per block over the last axis (float32, as a matrix product)."""
    zr = z.reshape(*z.shape[:-1], -1, block) @ matrix(block).T
    return zr.reshape(z.shape) * np.asarray(signs, np.float32)


def restored_bfp_rows(scales, codes, signs, block):
    """Rotated ternary embedding rows dequantized, restored to the plain basis (times the image
    gain) and quantized to int16 BFP rows: per row the exponent puts the absmax in [2^14, 2^15),
    mantissas rounded to nearest and clipped to +-32767 (model/bons.py:243-259)."""
    rows, cols = codes.shape
    z = (codes.astype(np.float32).reshape(rows, cols // L.GROUP, L.GROUP) - 1.0) \
        * np.asarray(scales).astype(np.float32)[:, :, None]
    e = (restore(z.reshape(rows, cols), signs, block) * np.float32(image_gain(block))).astype(np.float64)
    amax = np.abs(e).max(axis=1)
    exps = np.where(amax > 0, np.floor(np.log2(np.maximum(amax, 1e-30))).astype(np.int64) - 14, 0)
    mant = np.clip(np.round(e * 2.0 ** (-exps[:, None])), -32767, 32767)
    return mant.astype(np.int16), exps.astype(np.int32)


def rotation_specs(cfg):
    """The image's rotation tensors, one per (input width, block), in width order."""
    from .bons import TensorSpec
    block = cfg.hadamard_block
    H = sign_matrix(block)
    scale = image_scales(block)[0]
    specs = []
    for wi, width in enumerate(sorted(cfg.hadamard_signs)):
        s = np.asarray(cfg.hadamard_signs[width], np.float32)
        for b in range(width // block):
            codes = (H * s[b * block:(b + 1) * block][None, :] + 1).astype(np.uint8)
            specs.append(TensorSpec(f"had.{width}.{b}", L.ROLE_HADAMARD, L.hadamard_layer(wi, b),
                                    L.KIND_TERNARY, block, block,
                                    scales=np.full((block, block // L.GROUP), scale, np.float16),
                                    values=codes, flags=0))
    return specs


def image_rotation(img):
    """(block, scale, {width: signs float32}) of a BONS image's rotation, read from its rotation
    tensors (row 0 of a block is R_pm1[0] * s = s), or None for a plain-basis image."""
    h = img.header
    block = h["hadamard_block"]
    if not block:
        return None
    out, scale = {}, None
    for wi, width in enumerate(h["hadamard_widths"]):
        parts = []
        for b in range(width // block):
            e = img.find(L.ROLE_HADAMARD, L.hadamard_layer(wi, b))
            if e is None:
                raise ValueError(f"rotated image without its rotation block {b} of width {width}")
            sc, codes = img.entry_tensor(e)
            parts.append(np.asarray(codes[0], np.float32) - 1.0)
            scale = float(np.asarray(sc)[0, 0])
        out[width] = np.concatenate(parts)
    return block, scale, out
