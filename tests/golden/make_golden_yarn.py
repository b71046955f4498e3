"""Write tests/golden/golden_yarn.npz from the reference implementation: a YaRN-scaled RoPE case.

Run in the development container only (it imports the reference's Python model package from
/root/reference, which never travels with this repository):

    python tests/golden/make_golden_yarn.py

What it pins: the RoPE of an image whose table carries YaRN scaling (model/golden.py:189-213,
baked into the image as Q14 rows by model/bons.py:356-367, read back per position by
model/mirror.py:478-483). The model is the tiny dense configuration with yarn_factor 4 over an
original context of 32, so positions past 32 rotate with the ramped frequencies and the
attention scale mscale = 1 + 0.1 ln 4. Stored:
  * the sha256 of the reference writer's image of this repository's synthetic tensors (this
    repository's writer must produce the same bytes, rope table included);
  * golden.FloatModel's logits (float64 YaRN tables, no Q14 rounding) at ten positions of a
    96-token sequence (a 16-token prompt and FloatModel's greedy continuation), and the sequence;
  * fastref.HybridRef's logits on the same image (plain RoPE: HybridRef ignores the table), to
    show the two differ.
Only inputs and outputs are stored; no reference source is copied.
"""

import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
REF = "/root/reference"

YARN_FACTOR, YARN_ORIG_CTX, SEED, N_PROMPT, N_SEQ = 4.0, 32, 5, 16, 96


def yarn_config():
    from trixium_amd import configs as C
    return C.TINY.replace(name="tiny-yarn", yarn_factor=YARN_FACTOR, yarn_orig_ctx=YARN_ORIG_CTX, max_ctx=128)


def main():
    from trixium_amd import layout as L, synth
    sys.path.insert(0, REF)
    from model import bons as rbons, configs as rconfigs, fastref, golden

    cfg = yarn_config()
    fields = {k: getattr(cfg, k) for k in rconfigs.ModelConfig.__dataclass_fields__}
    rcfg = rconfigs.ModelConfig(**fields)
    specs = synth.small_model_tensors(cfg, SEED, True)
    rspecs = [rbons.TensorSpec(s.name, s.role, s.layer, s.kind, s.rows, s.cols, scales=s.scales,
                               values=s.values, flags=s.flags) for s in specs]
    p = os.path.join(tempfile.mkdtemp(), "yarn.img")
    rbons.write_image(rcfg, rspecs, 1, p, trit5=True)
    sha = hashlib.sha256(open(p, "rb").read()).hexdigest()

    tensors = {}
    for s in specs:
        if s.kind == L.KIND_TERNARY:
            w = (s.values.astype(np.float32).reshape(s.rows, -1, 128) - 1.0) * s.scales.astype(np.float32)[:, :, None]
            tensors[s.name] = w.reshape(s.rows, s.cols)
        elif s.kind == L.KIND_F32:
            if s.role == L.ROLE_LM_HEAD:
                tensors[s.name] = s.values
                tensors["token_embd.weight"] = s.values
            else:
                tensors[s.name] = s.values.reshape(-1)

    fm = golden.FloatModel(rcfg, tensors)
    prompt = synth.random_prompt(cfg, N_PROMPT, SEED)
    seq = list(prompt)
    logits = [fm.forward(prompt)]
    while len(seq) < N_SEQ:
        seq.append(int(np.argmax(logits[-1])))
        logits.append(fm.forward([seq[-1]]))
    seq = np.array(seq, np.int32)
    pos = np.array([N_PROMPT - 1, N_PROMPT, 24, 31, 32, 40, 56, 72, 88, N_SEQ - 1], np.int32)
    fm_logits = np.stack(logits).astype(np.float32)[pos - (N_PROMPT - 1)]

    ref = fastref.HybridRef(rbons.BONSReader(p))
    fr_logits = ref.logits(ref.hidden(list(seq)))[pos].astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "golden_yarn.npz"), image_sha256=np.frombuffer(sha.encode(), np.uint8),
                        seq=seq, n_prompt=np.int32(N_PROMPT), pos=pos, floatmodel_logits=fm_logits,
                        fastref_logits=fr_logits)
    d = np.abs(fm_logits - fr_logits).max() / np.abs(fm_logits).max()
    print("image", sha, "floatmodel vs fastref (plain RoPE) rel diff", d)


if __name__ == "__main__":
    main()
