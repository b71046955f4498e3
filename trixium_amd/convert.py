"""GGUF (PrismML Bonsai: PQ2_0 / g128 Q2_0 / PTQ1_0 / Q1_0 ternary) -> BONS image.

The conversion of model/convert.py:120-343 for the images this decoder reads:
- the model config from the GGUF metadata (model/golden.py:45-101);
- every tensor by its GGUF name to a (role, layer, replicated) entry, in the reference's
  canonical order (embedding, each layer's tensors, final norm, head);
- ternary blocks decoded to codes 0..2 with their fp16 group scales (1-bit weights as codes 0/2);
  the codes load one tensor at a time while the image is written;
- row-sharded vocabulary tensors padded with zero-weight rows (code 1, scale 0) to a multiple of
  the channel count;
- the DeltaNet beta/alpha head projections (F32 or BF16) requantised to Q8 rows (absmax/127 per
  32 weights, fp16 scales, round half to even); Q8_0 tensors taken as they are; F32 tensors as
  F32 rows (the conv taps as rows of 1024);
- matrices wider than kseg_max split into K-segments;
- written with write_image (rope table, int16 embedding table, optional trit5 storage);
- PrismML's Hadamard-rotated files: the rotation tensors of every input width, the odd-block
  scale fold, and the token table restored to the plain basis in the int16 embedding table.

Not done here: the FPGA board's channel-window fit check (model/convert.py:260-312: HBM windows,
per-channel KV and DeltaNet budgets), which can drop the int16 embedding table for an FPGA
image.

    python -m trixium_amd.convert inspect FILE.gguf
    python -m trixium_amd.convert convert --gguf F --channels 1 --out IMG [--trit5] [--check] ...
    python -m trixium_amd.convert verify --image IMG
"""

import argparse
import hashlib
import sys
import time

import numpy as np

from . import hadamard
from . import layout as L
from . import qformats as Q
from .bons import BONSReader, TensorSpec, split_wide, write_image
from .configs import ModelConfig
from .gguf import GGUFReader, inspect as gguf_inspect

ARCHS = ("qwen3", "qwen35", "qwen3next")

# GGUF tensor name -> (role, replicated), model/convert.py:41-71.
GLOBAL_ROLES = {
    "token_embd.weight": (L.ROLE_TOK_EMB, False),
    "output_norm.weight": (L.ROLE_OUT_NORM, True),
    "output.weight": (L.ROLE_LM_HEAD, False),
}
BLOCK_ROLES = {
    "attn_norm": (L.ROLE_ATTN_NORM, True),
    "attn_q": (L.ROLE_ATTN_Q, False),
    "attn_k": (L.ROLE_ATTN_K, False),
    "attn_v": (L.ROLE_ATTN_V, False),
    "attn_q_norm": (L.ROLE_ATTN_Q_NORM, True),
    "attn_k_norm": (L.ROLE_ATTN_K_NORM, True),
    "attn_output": (L.ROLE_ATTN_OUT, False),
    "ffn_norm": (L.ROLE_FFN_NORM, True),
    "ffn_gate": (L.ROLE_FFN_GATE, False),
    "ffn_up": (L.ROLE_FFN_UP, False),
    "ffn_down": (L.ROLE_FFN_DOWN, False),
    "post_attention_norm": (L.ROLE_FFN_NORM, True),     # Qwen3.5's name of the FFN input norm
    "attn_qkv": (L.ROLE_ATTN_QKV, False),
    "attn_gate": (L.ROLE_ATTN_ZGATE, False),
    "ssm_out": (L.ROLE_SSM_OUT, False),
    "ssm_beta": (L.ROLE_SSM_BETA, False),
    "ssm_alpha": (L.ROLE_SSM_ALPHA, False),
    "ssm_conv1d": (L.ROLE_SSM_CONV, True),
    "ssm_a": (L.ROLE_SSM_A, True),
    "ssm_dt": (L.ROLE_SSM_DT, True),
    "ssm_norm": (L.ROLE_SSM_NORM, True),
}
# Per-layer tensor order of a Qwen3 attention layer, a Qwen3.5 attention layer and a Qwen3.5
# Gated DeltaNet layer (model/convert.py:73-81).
ATTN_TENSORS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_q_norm", "attn_k_norm",
                "attn_output", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")
ATTN_TENSORS_Q35 = ATTN_TENSORS[:7] + ("post_attention_norm",) + ATTN_TENSORS[8:]
DN_TENSORS = ("attn_norm", "attn_qkv", "attn_gate", "ssm_beta", "ssm_alpha", "ssm_conv1d",
              "ssm_a", "ssm_dt", "ssm_norm", "ssm_out", "post_attention_norm", "ffn_gate",
              "ffn_up", "ffn_down")
TERNARY_TYPES = (Q.GGML_Q2_0, Q.GGML_PQ2_0, Q.GGML_PTQ1_0, Q.GGML_Q1_0)


def config_from_gguf(reader):
    """ModelConfig from the GGUF metadata (model/golden.py:45-101)."""
    md = reader.metadata
    arch = md.get("general.architecture")
    if arch not in ARCHS:
        raise ValueError(f"unsupported architecture {arch!r} (known: {ARCHS})")

    def g(key, default=None):
        return md.get(f"{arch}.{key}", default)

    name = str(md.get("general.basename", arch)).lower()
    if name in ("folded", "hf", "") and md.get("general.size_label"):
        name = f"bonsai-{str(md['general.size_label']).lower()}"
    n_embd, n_head = int(g("embedding_length")), int(g("attention.head_count"))
    cfg = ModelConfig(
        name=name, n_layer=int(g("block_count")), n_embd=n_embd, n_head=n_head,
        n_kv_head=int(g("attention.head_count_kv")),
        head_dim=int(g("attention.key_length", n_embd // n_head)),
        ffn_dim=int(g("feed_forward_length")), vocab=reader.tensors["token_embd.weight"].shape[0],
        rope_theta=float(g("rope.freq_base", 10000.0)),
        rms_eps=float(g("attention.layer_norm_rms_epsilon", 1e-6)),
        tie_embeddings="output.weight" not in reader.tensors,
        yarn_factor=float(g("rope.scaling.factor", 1.0)) if g("rope.scaling.type") == "yarn" else 1.0,
        yarn_orig_ctx=int(g("rope.scaling.original_context_length", 0)))
    if arch in ("qwen35", "qwen3next"):
        every = int(g("full_attention_interval", 4))
        cfg.layer_types = tuple("attn" if (l + 1) % every == 0 else "deltanet" for l in range(cfg.n_layer))
        cfg.dn_num_v_heads = int(g("ssm.time_step_rank", 0))
        cfg.dn_num_k_heads = int(g("ssm.group_count", 0))
        cfg.dn_k_head_dim = int(g("ssm.state_size", 0))
        cfg.dn_v_head_dim = int(g("ssm.inner_size", 0)) // max(1, cfg.dn_num_v_heads)
        cfg.dn_conv_kernel = int(g("ssm.conv_kernel", 0))
        cfg.rope_dims = int(g("rope.dimension_count", 0))
        # attn_q holds [q | gate] when it has 2 q_dim rows (read from the first attention layer).
        first = next((l for l in range(cfg.n_layer) if cfg.layer_types[l] == "attn"), None)
        q = reader.tensors.get(f"blk.{first}.attn_q.weight") if first is not None else None
        if q is not None:
            cfg.attn_gated = q.shape[0] == 2 * cfg.q_dim
    if md.get("prism.hadamard.block_size"):
        if md.get("prism.hadamard.transform") != "normalized-sylvester-walsh-hadamard" or \
                md.get("prism.hadamard.axis") != "input-last-dimension":
            raise ValueError("unknown prism.hadamard transform or axis")
        cfg.hadamard_block = int(md["prism.hadamard.block_size"])
        widths, signs = md["prism.hadamard.sign_widths"], md["prism.hadamard.sign_values"]
        cfg.hadamard_signs, at = {}, 0
        for w in widths:
            cfg.hadamard_signs[int(w)] = tuple(int(v) for v in signs[at:at + int(w)])
            at += int(w)
        if at != len(signs):
            raise ValueError(f"hadamard signs: {len(signs)} values for widths summing to {at}")
    return cfg


def check_engine_support(cfg):
    """SystemExit when a width is not a whole number of 128-weight groups (model/golden.py:103-108)."""
    for name, dim in (("n_embd", cfg.n_embd), ("ffn_dim", cfg.ffn_dim), ("head_dim", cfg.head_dim)):
        if dim % L.GROUP:
            raise SystemExit(f"{cfg.name}: {name} = {dim} is not a multiple of the 128-wide ternary group")


def name_role(name):
    """(layer, role, replicated) of a GGUF tensor name."""
    if name in GLOBAL_ROLES:
        return (0,) + GLOBAL_ROLES[name]
    if name.startswith("blk."):
        _, layer, base = name.split(".", 2)
        for suffix in (".weight", ".bias"):
            if base.endswith(suffix):
                base = base[:-len(suffix)]
        return (int(layer),) + BLOCK_ROLES[base]
    raise KeyError(name)


def _q2_group(raw, n, align):
    """Which block a type-42 payload holds: q2_0_group on its size, else the one block size the
    file's alignment padding after the tensor allows."""
    try:
        return Q.q2_0_group(raw, n)
    except ValueError:
        fit = [g for g, size in ((128, n // 128 * Q.BLOCK_Q2_0), (64, n // 64 * 18))
               if size <= raw.size < size + align]
        if len(fit) != 1:
            raise
        return fit[0]


def _ternary_source(reader, name, t):
    """(scales fp16 flat, code loader) of a ternary-block tensor."""
    raw = reader.tensor_bytes(name)
    n = t.n_elements
    if t.type_id == Q.GGML_Q2_0:
        if _q2_group(raw, n, int(reader.metadata.get("general.alignment", 32))) != 128:
            raise NotImplementedError(f"{name}: group-64 Q2_0 (two scales per 128 weights) does not fit "
                                      "the 128-group rows; convert the PQ2_0 file of the model")
        raw = raw[:n // 128 * Q.BLOCK_Q2_0]
    if t.type_id in (Q.GGML_Q2_0, Q.GGML_PQ2_0):
        return Q.q2_0_scales(raw), lambda: Q.q2_0_unpack(raw)[1]
    if t.type_id == Q.GGML_PTQ1_0:
        return Q.ptq1_0_scales(raw), lambda: Q.ptq1_0_unpack(raw)[1]
    return Q.q1_0_unpack(raw)[0], lambda: Q.q1_0_to_ternary_codes(raw)[1]


def q8_rows(name, role, layer, w):
    """A float matrix as Q8 rows: fp16 scale amax/127 per 32 weights, q = round(w / scale) (half to
    even), clipped to +-127 (model/convert.py:191-202)."""
    rows, cols = w.shape
    grp = np.asarray(w, np.float32).reshape(rows, cols // L.GROUP_Q8, L.GROUP_Q8)
    scales = (np.abs(grp).max(axis=2) / 127.0).astype(np.float16)
    sc = scales.astype(np.float32)[:, :, None]
    q = np.rint(np.divide(grp, sc, out=np.zeros_like(grp), where=sc > 0)).clip(-127, 127)
    return TensorSpec(name, role, layer, L.KIND_Q8, rows, cols, scales=scales,
                      values=q.reshape(rows, cols).astype(np.int8), flags=0)


def spec_from_gguf(reader, name, n_channels, vocab_pad):
    """The image entry of one GGUF tensor (model/convert.py:120-189)."""
    t = reader.tensors[name]
    layer, role, repl = name_role(name)
    flags = L.FLAG_REPLICATED if repl else 0
    if t.type_id in TERNARY_TYPES:
        rows, cols = t.shape
        scales, unpack = _ternary_source(reader, name, t)
        scales = scales.reshape(rows, cols // L.GROUP)
        pad = 0
        if not repl and rows % n_channels:
            if role not in (L.ROLE_TOK_EMB, L.ROLE_LM_HEAD):
                raise ValueError(f"{name}: {rows} rows do not shard over {n_channels} channels")
            pad = vocab_pad - rows
            scales = np.concatenate([scales, np.zeros((pad, scales.shape[1]), np.float16)])

        def load(unpack=unpack, rows=rows, cols=cols, pad=pad):
            codes = unpack().reshape(rows, cols)
            return np.concatenate([codes, np.ones((pad, cols), np.uint8)]) if pad else codes
        return TensorSpec(name, role, layer, L.KIND_TERNARY, rows + pad, cols, scales=scales,
                          loader=load, flags=flags)
    raw = reader.tensor_bytes(name)
    if role in (L.ROLE_SSM_BETA, L.ROLE_SSM_ALPHA) and t.type_name in ("F32", "BF16"):
        deq = Q.f32_dequant if t.type_name == "F32" else Q.bf16_dequant
        return q8_rows(name, role, layer, deq(raw).reshape(t.shape))
    if t.type_name == "F32":
        v = Q.f32_dequant(raw).reshape(t.shape)
        v = v.reshape(1, -1) if v.ndim == 1 else v
        if role == L.ROLE_SSM_CONV:
            v = v.reshape(-1, 1024)          # tap i of channel c at flat index c * taps + i
        return TensorSpec(name, role, layer, L.KIND_F32, v.shape[0], v.shape[1], values=v,
                          flags=L.FLAG_REPLICATED)
    if t.type_name == "Q8_0":
        rows, cols = t.shape
        blk = np.asarray(raw).reshape(rows, cols // Q.QK_Q8_0, Q.BLOCK_Q8_0)
        return TensorSpec(name, role, layer, L.KIND_Q8, rows, cols,
                          scales=np.ascontiguousarray(blk[:, :, :2]).view(np.float16).reshape(rows, -1),
                          values=np.ascontiguousarray(blk[:, :, 2:]).view(np.int8).reshape(rows, cols),
                          flags=flags)
    raise NotImplementedError(f"{name}: tensor type {t.type_name} is not converted")


def tensor_names(reader, cfg):
    """The image's tensor order: embedding, each layer's tensors, final norm, head."""
    names = ["token_embd.weight"]
    for l in range(cfg.n_layer):
        if cfg.layer_type(l) == "deltanet":
            bases = DN_TENSORS
        elif f"blk.{l}.post_attention_norm.weight" in reader.tensors:
            bases = ATTN_TENSORS_Q35
        else:
            bases = ATTN_TENSORS
        for b in bases:
            names.append(f"blk.{l}.{b}" + (".bias" if b == "ssm_dt" else "" if b == "ssm_a" else ".weight"))
    names.append("output_norm.weight")
    if "output.weight" in reader.tensors:
        names.append("output.weight")
    return names


def convert(gguf_path, n_channels, out_path, manifest_path=None, tokenizer_path=None,
            max_layers=None, check=False, emb16=True, kseg_max=L.KSEG_MAX, trit5=False, log=print):
    """Write the BONS image of a GGUF file; returns the manifest."""
    reader = GGUFReader(gguf_path)
    cfg = config_from_gguf(reader)
    try:
        check_engine_support(cfg)
    except SystemExit as e:
        log(f"  NOTE: {e}")
    if max_layers is not None:
        cfg.n_layer = min(cfg.n_layer, max_layers)
        cfg.name = f"{cfg.name}-l{cfg.n_layer}"
    vocab_pad = cfg.vocab_padded(n_channels)
    specs = [spec_from_gguf(reader, n, n_channels, vocab_pad) for n in tensor_names(reader, cfg)]
    if cfg.hadamard_block:
        # An odd power-of-two block: the rotation tensors carry 2^-floor(k/2), so every rotated
        # ternary tensor (the projections, the head and the token table) takes the remaining
        # 2^-0.5 in its scales. As in model/convert.py:229-239 the fold comes after the entries'
        # bias/rshift were chosen from the unfolded scales.
        fold = hadamard.image_scales(cfg.hadamard_block)[1]
        if fold != 1.0:
            for sp in specs:
                if sp.kind == L.KIND_TERNARY:
                    sp.scales = (sp.scales.astype(np.float32) * np.float32(fold)).astype(np.float16)
            log(f"  hadamard block {cfg.hadamard_block}: weights x 2**-0.5")
        specs += hadamard.rotation_specs(cfg)
    specs = [seg for sp in specs for seg in split_wide(sp, kseg_max)]
    nseg = sum(1 for sp in specs if sp.flags & L.FLAG_KSEG)
    if nseg:
        log(f"  {nseg} K-segments (matrices wider than {kseg_max})")
    sha = b""
    if tokenizer_path:
        with open(tokenizer_path, "rb") as f:
            sha = hashlib.sha256(f.read()).digest()
    t0 = time.time()
    manifest = write_image(cfg, specs, n_channels, out_path, tokenizer_sha256=sha,
                           manifest_path=manifest_path, emb16=emb16, trit5=trit5)
    log(f"image: {out_path} {manifest['payload_beats'] * L.BEAT / 1e6:.1f} MB/channel x {n_channels} "
        f"channels ({time.time() - t0:.1f} s)")
    if check:
        img = BONSReader(out_path)
        first = next(n for n in ("blk.0.attn_q.weight", "blk.0.attn_qkv.weight") if any(s.name == n for s in specs))
        for name in (first, "blk.0.ffn_gate.weight"):
            s_img, v_img = img.tensor(name)
            sp = next(s for s in specs if s.name == name)
            if not (np.array_equal(v_img, sp.load()) and np.array_equal(s_img, sp.scales.astype(np.float16))):
                raise AssertionError(f"{name}: image tensor differs from the GGUF")
            log(f"  check {name}: OK")
    return manifest


def verify(image_path, log=print):
    """Re-check every entry's CRC over its channel payloads (model/convert.py:345-361)."""
    img = BONSReader(image_path)
    h = img.header
    bad = 0
    for e in img.entries:
        crc = 0
        for c in range(h["n_channels"]):
            crc = L.crc32(np.asarray(img.entry_channel_bytes(e, c)), crc)
        if crc != e["crc32"]:
            bad += 1
            log(f"  CRC MISMATCH {e['name']}: {crc:#x} != {e['crc32']:#x}")
    log("verify: OK" if not bad else f"verify: {bad} bad tensors")
    return bad == 0


def main(argv=None):
    ap = argparse.ArgumentParser(description="GGUF -> BONS converter")
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("inspect", help="print a GGUF file's metadata and tensors")
    p.add_argument("gguf")
    p = sub.add_parser("convert", help="write the BONS image of a GGUF file")
    p.add_argument("--gguf", required=True)
    p.add_argument("--channels", required=True, type=int)
    p.add_argument("--out", required=True)
    p.add_argument("--manifest", default=None)
    p.add_argument("--tokenizer", default=None)
    p.add_argument("--layers", default=None, type=int)
    p.add_argument("--check", action="store_true")
    p.add_argument("--no-emb16", action="store_true")
    p.add_argument("--kseg-max", default=L.KSEG_MAX, type=int)
    p.add_argument("--trit5", action="store_true")
    p = sub.add_parser("verify", help="re-check an image's CRCs")
    p.add_argument("--image", required=True)
    a = ap.parse_args(argv)
    if a.cmd == "inspect":
        gguf_inspect(a.gguf)
    elif a.cmd == "convert":
        convert(a.gguf, a.channels, a.out, a.manifest or a.out.rsplit(".", 1)[0] + ".json", a.tokenizer,
                a.layers, a.check, emb16=not a.no_emb16, kseg_max=a.kseg_max, trit5=a.trit5)
    else:
        return 0 if verify(a.image) else 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
