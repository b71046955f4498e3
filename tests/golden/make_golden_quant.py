"""Write tests/golden/golden_quant.npz from the reference implementation: the firmware's
activation quantizer and its quantized projection.

Run in the development container only (it imports the reference's Python model package from
/root/reference, which never travels with this repository):

    python tests/golden/make_golden_quant.py

What it pins: model/mirror.py:45-51 `_quantize_f_pow2` (with its float32 lroundf,
mirror.py:34-35) on edge-case vectors (halves that round away from zero, a maximum exactly at a
power of two and just below one, magnitudes far from 1, a lone nonzero, a mantissa that rounds
up to 128 and is clipped), and the engine path of mirror.py:663-678 (quantize, the reference's
bitexact.matvec_ternary with the tensor's B and R, the int32 result times 2^(e8 + R - B)) on
seeded ternary tensors. Only inputs and outputs are stored; no reference source is copied.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"
f32 = np.float32


def vectors():
    r = np.random.default_rng(17)
    vs = {
        "normal": r.standard_normal(2048).astype(f32),
        "halves": (np.arange(-20, 21, dtype=f32) + f32(0.5)) * f32(2.0**-3),
        "pow2_max": np.array([8.0, -3.0, 0.0625, 7.9375, -8.0, 1.0], f32),
        "below_pow2": np.array([np.nextafter(f32(4.0), f32(0.0)), 1.5, -0.75, 2.0**-20], f32),
        "tiny": (r.standard_normal(300) * 1e-30).astype(f32),
        "huge": (r.standard_normal(300) * 1e30).astype(f32),
        "lone": np.array([0.0, 0.0, -0.3, 0.0], f32),
        "round_to_128": np.array([127.6, 1.0, -127.6, 0.5], f32) * f32(2.0**-5),
        "zeros": np.zeros(64, f32),
    }
    vs["ties_low"] = np.array([f32(0.49999997), f32(-0.49999997), f32(64.0)], f32)
    vs["ties"] = np.array([100.0, 2.5, -2.5, 3.5, -0.5, 0.5, -126.5, 126.5], f32)
    return vs


def projections():
    out = []
    for i, (M, K) in enumerate(((64, 256), (300, 2048), (17, 640))):
        r = np.random.default_rng(100 + i)
        u = r.random((M, K))
        codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
        scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
        x = (r.standard_normal(K) * (3.0 if i == 1 else 0.2)).astype(f32)
        out.append((f"proj{i}", codes, scales, x))
    return out


def main():
    sys.path.insert(0, REF)
    from model import bitexact as rbx
    from model.mirror import _quantize_f_pow2
    arrays = {}
    for name, x in vectors().items():
        q, e = _quantize_f_pow2(x)
        arrays[f"q/{name}/x"], arrays[f"q/{name}/x8"], arrays[f"q/{name}/e8"] = x, q, np.int32(e)
    for name, codes, scales, x in projections():
        _, e16 = rbx.fp16_decompose(scales)
        B = rbx.choose_scale_bias(e16)
        R = rbx.choose_result_shift(scales, B)
        x8, e8 = _quantize_f_pow2(x)
        res = rbx.matvec_ternary(scales, codes, x8, B, R)
        y = res.astype(np.int32).astype(f32) * f32(np.exp2(f32(e8 + R - B)))
        arrays[f"p/{name}/B"], arrays[f"p/{name}/R"] = np.int32(B), np.int32(R)
        arrays[f"p/{name}/y"] = y.astype(f32)
    np.savez_compressed(os.path.join(HERE, "golden_quant.npz"), **arrays)
    print(len(arrays), "arrays")


if __name__ == "__main__":
    main()
