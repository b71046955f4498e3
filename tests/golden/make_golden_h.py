"""Write tests/golden/golden_h_geometry.npz from the reference implementation: a two-layer model
(one Gated DeltaNet layer, one gated attention layer) at the 27B hybrid's layer geometry
(width 5120, 24 q / 4 kv heads of 256 with 64 RoPE dims, 48 value / 16 key DeltaNet heads of 128,
FFN 17408), vocabulary 512, seed 7.

Run in the development container only (it imports the reference's Python model package from
/root/reference, which never travels with this repository):

    python tests/golden/make_golden_h.py

Stored (inputs and outputs only, no reference source):
  * image_sha256: the reference writer (model/bons.py:342-459) on this repository's synthetic
    tensors (trit5, one channel); this repository's writer must produce the same bytes;
  * prompt, the greedy tokens of HybridRef (model/fastref.py) and its logits at the last prompt
    position and the generated positions, with each position's top-2 logit margin.
It also prints the error of this repository's float oracle (oracle/floatref.py) against those
logits, which pins the oracle at this geometry.
"""

import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE) + "/..")
REF = "/root/reference"

SEED, N_PROMPT, N_NEW = 7, 6, 4


def h_config():
    from trixium_amd import configs as C
    return C.QWEN35_27B.replace(name="qwen3.5-27b-geometry-2l", n_layer=2, layer_types=("deltanet", "attn"),
                                vocab=512, max_ctx=64)


def main():
    from trixium_amd import bons, synth
    from trixium_amd import layout as L
    from oracle.floatref import FloatRef
    sys.path.insert(0, REF)
    from model import bons as rbons, configs as rconfigs, fastref

    cfg = h_config()
    fields = {k: getattr(cfg, k) for k in rconfigs.ModelConfig.__dataclass_fields__}
    rcfg = rconfigs.ModelConfig(**fields)
    specs = synth.small_model_tensors(cfg, SEED, True)
    rspecs = []
    for s in specs:
        kw = dict(scales=s.scales, values=s.values, flags=s.flags)
        if s.kind == L.KIND_NORM16:
            kw["bias"] = None
        rspecs.append(rbons.TensorSpec(s.name, s.role, s.layer, s.kind, s.rows, s.cols, **kw))
    tmp = tempfile.mkdtemp()
    p_ref, p_own = os.path.join(tmp, "ref.img"), os.path.join(tmp, "own.img")
    rbons.write_image(rcfg, rspecs, 1, p_ref, trit5=True)
    bons.write_image(cfg, specs, 1, p_own, trit5=True)
    sha_ref = hashlib.sha256(open(p_ref, "rb").read()).hexdigest()
    sha_own = hashlib.sha256(open(p_own, "rb").read()).hexdigest()
    print("image sha256", sha_ref, "own writer equal:", sha_ref == sha_own, flush=True)

    ref = fastref.HybridRef(rbons.BONSReader(p_ref))
    prompt = synth.random_prompt(cfg, N_PROMPT, SEED)
    seq = list(prompt)
    for _ in range(N_NEW):
        lg = ref.logits(ref.hidden(seq)[-1:])[0]
        seq.append(int(np.argmax(lg)))
        print("token", seq[-1], flush=True)
    lg_all = ref.logits(ref.hidden(seq))
    pos = list(range(N_PROMPT - 1, len(seq)))
    logits = lg_all[pos].astype(np.float32)
    top2 = np.sort(logits, axis=1)[:, -2:]
    margin = (top2[:, 1] - top2[:, 0]).astype(np.float32)

    own = FloatRef(bons.BONSReader(p_own))
    want = [own.forward(prompt)] + [own.step(t) for t in seq[N_PROMPT:]]
    err = max(float(np.max(np.abs(w - g)) / np.max(np.abs(g))) for w, g in zip(want, logits))
    print("oracle vs HybridRef max rel err", err, flush=True)

    np.savez(os.path.join(HERE, "golden_h_geometry.npz"),
             image_sha256=np.frombuffer(sha_ref.encode(), np.uint8), prompt=np.array(prompt, np.int32),
             tokens=np.array(seq[N_PROMPT:], np.int32), logits_pos=np.array(pos, np.int32), logits=logits,
             top2_margin=margin, oracle_rel_err=np.float32(err))
    print("wrote", os.path.join(HERE, "golden_h_geometry.npz"))


if __name__ == "__main__":
    main()
