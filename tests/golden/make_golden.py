"""Write the golden fixtures under tests/golden/ from the reference implementation.

Run in the development container only (it imports the reference's Python model package from
/root/reference, which never travels with this repository):

    python tests/golden/make_golden.py

What it pins, for the functions no closed form or reference test pins:
  * image bytes: the reference writer (model/bons.py:342-459) on this repository's synthetic
    tensors, trit5 and 2-bit, 1 and 2 channels -> sha256 of each image;
  * HybridRef (model/fastref.py) teacher-forced logits and its greedy tokens on the tiny dense
    and tiny hybrid models;
  * FloatModel.generate (model/golden.py:462-470) and hybrid27_generate(exact=True)
    (model/mirror.py:594) tokens on the same models;
  * embed_bfp_rows (model/bons.py:204-236) on edge-case rows;
  * matvec_ternary (model/bitexact.py:101-119) on the four microbench shapes: sha256 of the
    int32 result plus a slice.
Only inputs and outputs are stored (npz/json); no reference source is copied.
"""

import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
REF = "/root/reference"


def sha(path_or_bytes):
    if isinstance(path_or_bytes, (bytes, bytearray)):
        return hashlib.sha256(path_or_bytes).hexdigest()
    with open(path_or_bytes, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def main():
    from trixium_amd import configs as C, synth
    from trixium_amd import layout as L
    sys.path.insert(0, REF)
    from model import bons as rbons, configs as rconfigs, fastref, golden, bitexact as rbx
    from model.mirror import hybrid27_generate

    out = {}
    arrays = {}

    def ref_cfg(cfg):
        fields = {k: getattr(cfg, k) for k in rconfigs.ModelConfig.__dataclass_fields__}
        return rconfigs.ModelConfig(**fields)

    def ref_specs(specs):
        res = []
        for s in specs:
            kw = dict(scales=s.scales, values=s.values, flags=s.flags)
            if s.kind == L.KIND_NORM16:
                kw["bias"] = None
            res.append(rbons.TensorSpec(s.name, s.role, s.layer, s.kind, s.rows, s.cols, **kw))
        return res

    def float_tensors(cfg, specs):
        """GGUF-named fp32 dict for FloatModel from the specs (dequantised)."""
        t = {}
        for s in specs:
            if s.kind == L.KIND_TERNARY:
                w = (s.values.astype(np.float32).reshape(s.rows, -1, 128) - 1.0) * s.scales.astype(np.float32)[:, :, None]
                t[s.name] = w.reshape(s.rows, s.cols)
            elif s.kind == L.KIND_Q8:
                w = s.values.astype(np.float32).reshape(s.rows, -1, 32) * s.scales.astype(np.float32)[:, :, None]
                t[s.name] = w.reshape(s.rows, s.cols)
            elif s.kind == L.KIND_F32:
                v = s.values
                if s.role == L.ROLE_SSM_CONV:
                    t[s.name] = v.reshape(-1, cfg.dn_conv_kernel)
                elif s.role == L.ROLE_LM_HEAD:
                    t[s.name] = v
                    t["token_embd.weight"] = v
                else:
                    t[s.name] = v.reshape(-1)
        return t

    tmp = tempfile.mkdtemp()
    # 1. Images: byte-exact writer parity ------------------------------------------------------
    images = {}
    for cfg, seed, fp16e in ((C.TINY, 0, True), (C.TINY_HYBRID, 1, True)):
        for trit5 in (True, False):
            for nch in (1, 2):
                specs = synth.small_model_tensors(cfg, seed, fp16e)
                p = os.path.join(tmp, f"{cfg.name}-t{int(trit5)}-n{nch}.img")
                rbons.write_image(ref_cfg(cfg), ref_specs(specs), nch, p, trit5=trit5)
                images[(cfg.name, trit5, nch)] = p
                out[f"image_sha256/{cfg.name}/trit5={int(trit5)}/n{nch}"] = sha(p)
    # A ternary tied embedding variant (the real models' layout, emb16 derived by the writer).
    specs = synth.small_model_tensors(C.TINY, 3, fp16_embedding=False)
    p = os.path.join(tmp, "tiny-ternemb.img")
    rbons.write_image(ref_cfg(C.TINY), ref_specs(specs), 1, p, trit5=True)
    out["image_sha256/tiny-ternemb/trit5=1/n1"] = sha(p)
    images[("tiny-ternemb", True, 1)] = p

    # 2./3. Logits and tokens -------------------------------------------------------------------
    for cfg, seed, key, n_new in ((C.TINY, 0, (C.TINY.name, True, 1), 64),
                                  (C.TINY_HYBRID, 1, (C.TINY_HYBRID.name, True, 1), 24),
                                  (C.TINY, 3, ("tiny-ternemb", True, 1), 32)):
        img = rbons.BONSReader(images[key])
        ref = fastref.HybridRef(img)
        prompt = synth.random_prompt(cfg, 16, seed)
        seq = list(prompt)
        for _ in range(n_new):                       # greedy, teacher-forced from position 0
            lg = ref.logits(ref.hidden(seq)[-1:])[0]
            seq.append(int(np.argmax(lg)))
        lg_all = ref.logits(ref.hidden(seq))
        name = key[0]
        out[f"fastref_tokens/{name}"] = seq[len(prompt):]
        out[f"prompt/{name}"] = prompt
        pos = sorted(set([len(prompt) - 1, len(prompt), len(prompt) + 7, len(seq) - 2, len(seq) - 1]))
        arrays[f"fastref_logits_pos/{name}"] = np.array(pos, np.int32)
        arrays[f"fastref_logits/{name}"] = lg_all[pos].astype(np.float32)
        top2 = np.sort(lg_all, axis=1)[:, -2:]
        out[f"fastref_min_top2_margin/{name}"] = float((top2[len(prompt) - 1:, 1] - top2[len(prompt) - 1:, 0]).min())
        fp16e = name != "tiny-ternemb"
        specs = synth.small_model_tensors(cfg, seed, fp16e)
        if fp16e:
            fm = golden.FloatModel(ref_cfg(cfg), float_tensors(cfg, specs))
            out[f"floatmodel_tokens/{name}"] = fm.generate(prompt, min(n_new, 24))
        if cfg.layer_types:
            out[f"mirror_exact_tokens/{name}"] = hybrid27_generate(img, prompt, 8, exact=True)

    # 4. embed_bfp_rows on edge rows -------------------------------------------------------------
    rng = np.random.default_rng(7)
    n, cols = 48, 256
    codes = rng.integers(0, 3, size=(n, cols)).astype(np.uint8)
    scales = np.exp2(rng.uniform(-14, 4, size=(n, cols // 128))).astype(np.float16)
    scales *= rng.choice([-1.0, 1.0], size=(n, cols // 128)).astype(np.float16)
    codes[0, :128] = 1
    codes[1, :] = 1
    scales[2, :] = np.float16(2.0**-6)
    scales[3, 0] = np.float16(2.0**-14); scales[3, 1:] = np.float16(8.0)
    scales[4, 0] = np.float16(2.0**-14); codes[4, 128:] = 1
    scales[5, :] = np.float16(1.0)
    from types import SimpleNamespace
    mant, exps = rbons.embed_bfp_rows(SimpleNamespace(values=codes, scales=scales))
    arrays["emb16_codes"], arrays["emb16_scales"] = codes, scales
    arrays["emb16_mant"], arrays["emb16_exp"] = mant, exps

    # 5. matvec_ternary on the microbench shapes -------------------------------------------------
    for (M, K) in C.MICROBENCH_SHAPES:
        r = np.random.default_rng(M * 7919 + K)
        u = r.random((M, K))
        cd = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
        sc = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
        x8 = r.integers(-127, 128, K, dtype=np.int8)
        _, e16 = rbx.fp16_decompose(sc)
        B = rbx.choose_scale_bias(e16)
        R = rbx.choose_result_shift(sc, B)
        res = rbx.matvec_ternary(sc, cd, x8, B, R)
        out[f"matvec/{M}x{K}"] = {"B": B, "R": R, "sha256": sha(res.astype("<i4").tobytes()),
                                  "head": res[:8].tolist()}

    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    np.savez_compressed(os.path.join(HERE, "golden_arrays.npz"), **arrays)
    print(json.dumps({k: v for k, v in out.items() if "margin" in k}, indent=1))


if __name__ == "__main__":
    main()
