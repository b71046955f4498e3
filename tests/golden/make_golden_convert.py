"""Write tests/golden/golden_convert.json: sha256 of the BONS images the reference's converter
(model/convert.py:convert) makes from the synthetic GGUF files of tests/synth_gguf.py:CASES:
  * qwen3, tiny shape, vocab 2048, one channel, 2-bit rows;
  * qwen3, tiny shape, vocab 1001 (padded to 1002), two channels, trit5 rows;
  * qwen35 hybrid (three Gated DeltaNet layers + one gated attention layer), trit5 rows, matrices
    wider than 256 split into K-segments;
and of ROT_CASES, PrismML-rotated files (qwen3 with 128-blocks, the hybrid with 256-blocks), for
which tests/golden/golden_rot_logits.npz also holds the logits of the reference's HybridRef
(model/fastref.py) on the reference's image at every position of an 8-token prompt.
Run in the development container only (it imports the reference from /root/reference, which never
travels with this repository):

    python tests/golden/make_golden_convert.py

It also converts the same files with trixium_amd.convert and prints whether the images match.
"""

import contextlib
import hashlib
import io
import json
import os
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "tests")]
REF = "/root/reference"

import synth_gguf                                    # noqa: E402
from synth_gguf import CASES, ROT_CASES              # noqa: E402
from trixium_amd import synth                        # noqa: E402
from trixium_amd import convert as own               # noqa: E402

def sha(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def main():
    sys.path.insert(0, REF)
    import numpy as np
    from model import bons as rbons, convert as ref, fastref
    out, logits, tmp = {}, {}, tempfile.mkdtemp()
    for c in CASES + ROT_CASES:
        g = os.path.join(tmp, c["id"] + ".gguf")
        synth_gguf.build(g, c["cfg"], c["seed"], c["arch"], hadamard=c.get("hadamard", 0))
        r_img, o_img = os.path.join(tmp, c["id"] + ".ref.bons"), os.path.join(tmp, c["id"] + ".own.bons")
        with contextlib.redirect_stdout(io.StringIO()):
            ref.convert(g, c["channels"], r_img, kseg_max=c["kseg_max"], trit5=c["trit5"])
        own.convert(g, c["channels"], o_img, kseg_max=c["kseg_max"], trit5=c["trit5"], log=lambda *a: None)
        out[c["id"]] = {"gguf_sha256": sha(g), "image_sha256": sha(r_img)}
        print(c["id"], "reference", sha(r_img)[:16], "own equal:", sha(r_img) == sha(o_img), flush=True)
        if c.get("hadamard"):
            hr = fastref.HybridRef(rbons.BONSReader(r_img))
            prompt = synth.random_prompt(c["cfg"], 8, c["seed"])
            logits[c["id"] + "/prompt"] = np.array(prompt, np.int32)
            logits[c["id"] + "/logits"] = hr.logits(hr.hidden(prompt)).astype(np.float32)
    with open(os.path.join(HERE, "golden_convert.json"), "w") as f:
        json.dump(out, f, indent=1)
    np.savez(os.path.join(HERE, "golden_rot_logits.npz"), **logits)
    print("wrote", os.path.join(HERE, "golden_convert.json"))


if __name__ == "__main__":
    main()
