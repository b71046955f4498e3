"""Write tests/golden/golden_score.npz from the reference implementation: HybridRef.score.

Run in the development container only (it imports the reference's Python model package from
/root/reference, which never travels with this repository):

    python tests/golden/make_golden_score.py

What it pins: model/fastref.py:244-273 `hidden` (the final normed hidden states) and `score`
(the next-token negative log-likelihoods, float64 log-sum-exp) on the tiny dense and tiny hybrid
fixture models (this repository's synthetic tensors written by the reference writer), over the
16-token fixture prompt followed by 24 tokens of a seeded random sequence. Stored: the tokens,
all T-1 NLLs and the hidden states at four positions. Only inputs and outputs are stored; no
reference source is copied.
"""

import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
REF = "/root/reference"

CASES = (("tiny-qwen3", 0), ("tiny-hybrid", 1))
HID_POS = (0, 15, 27, 39)


def sequence(cfg, seed):
    from trixium_amd import synth
    rest = np.random.default_rng(seed + 100).integers(0, cfg.vocab, 24)
    return synth.random_prompt(cfg, 16, seed) + [int(t) for t in rest]


def main():
    from trixium_amd import configs as C, synth
    sys.path.insert(0, REF)
    from model import bons as rbons, configs as rconfigs, fastref

    arrays = {}
    for name, seed in CASES:
        cfg = C.TINY if name == "tiny-qwen3" else C.TINY_HYBRID
        fields = {k: getattr(cfg, k) for k in rconfigs.ModelConfig.__dataclass_fields__}
        specs = synth.small_model_tensors(cfg, seed, True)
        rspecs = [rbons.TensorSpec(s.name, s.role, s.layer, s.kind, s.rows, s.cols, scales=s.scales,
                                   values=s.values, flags=s.flags) for s in specs]
        p = os.path.join(tempfile.mkdtemp(), name + ".img")
        rbons.write_image(rconfigs.ModelConfig(**fields), rspecs, 1, p, trit5=True)
        seq = sequence(cfg, seed)
        nll, hs = fastref.HybridRef(rbons.BONSReader(p)).score(seq)
        arrays[f"{name}/tokens"] = np.array(seq, np.int32)
        arrays[f"{name}/nll"] = np.asarray(nll, np.float64)
        arrays[f"{name}/hidden_pos"] = np.array(HID_POS, np.int32)
        arrays[f"{name}/hidden"] = np.asarray(hs, np.float32)[list(HID_POS)]
        print(name, "mean nll", float(np.mean(nll)))
    np.savez_compressed(os.path.join(HERE, "golden_score.npz"), **arrays)


if __name__ == "__main__":
    main()
