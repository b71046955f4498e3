"""Synthetic Bonsai-style GGUF files for the converter tests: the seeded small-model tensors of
trixium_amd.synth written in the PrismML block formats, the ternary matrices cycling through
PTQ1_0, PQ2_0 and the g128 type-42 Q2_0, one 1-bit (Q1_0) matrix, the DeltaNet beta in Q8_0 and
alpha in BF16, everything else F32. Shapes keep every payload but the embedding a multiple of the
32-byte alignment, as in real files."""

import numpy as np

from trixium_amd import configs as C, layout as L, qformats as Q, synth
from trixium_amd.gguf import T_ARR, T_F32, T_I8, T_I32, T_STR, Typed, write_gguf

TERNARY_CYCLE = (Q.GGML_PTQ1_0, Q.GGML_PQ2_0, Q.GGML_Q2_0)

# The converter's golden cases: qwen3 tiny shape on one channel in 2-bit rows; qwen3 with an odd
# vocabulary (padded) on two channels in trit5 rows; the qwen35 hybrid (three Gated DeltaNet
# layers, one gated attention layer) in trit5 rows with matrices wider than 256 split.
CASES = [
    {"id": "qwen3_ch1", "cfg": C.TINY.replace(name="tiny-gguf"), "arch": "qwen3", "seed": 3, "channels": 1,
     "trit5": False, "kseg_max": 16384},
    {"id": "qwen3_ch2_vocab1001", "cfg": C.TINY.replace(name="tiny-gguf", vocab=1001), "arch": "qwen3", "seed": 4,
     "channels": 2, "trit5": True, "kseg_max": 16384},
    {"id": "qwen35_hybrid_kseg", "cfg": C.TINY_HYBRID.replace(name="tiny-hybrid-gguf"), "arch": "qwen35",
     "seed": 5, "channels": 1, "trit5": True, "kseg_max": 256},
]
# PrismML-rotated files: qwen3 with 128-blocks (an odd power of two: the converter folds 2^-0.5
# into the weights) and the hybrid with 256-blocks.
ROT_CASES = [
    {"id": "qwen3_rot128", "cfg": C.TINY.replace(name="tiny-gguf-rot"), "arch": "qwen3", "seed": 6, "channels": 1,
     "trit5": True, "kseg_max": 16384, "hadamard": 128},
    {"id": "qwen35_rot256", "cfg": C.TINY_HYBRID.replace(name="tiny-hybrid-gguf-rot"), "arch": "qwen35", "seed": 7,
     "channels": 1, "trit5": True, "kseg_max": 16384, "hadamard": 256},
]


def input_widths(cfg):
    """The input widths of the model's ternary projections (what a rotation must cover)."""
    w = {cfg.n_embd, cfg.q_dim, cfg.ffn_dim}
    if any(cfg.layer_type(l) == "deltanet" for l in range(cfg.n_layer)):
        w.add(cfg.dn_num_v_heads * cfg.dn_v_head_dim)
    return sorted(w)


def _meta(cfg, arch):
    a = arch
    md = {"general.architecture": a, "general.basename": cfg.name, "general.size_label": "tiny",
          f"{a}.block_count": cfg.n_layer, f"{a}.context_length": 4096,
          f"{a}.embedding_length": cfg.n_embd, f"{a}.feed_forward_length": cfg.ffn_dim,
          f"{a}.attention.head_count": cfg.n_head, f"{a}.attention.head_count_kv": cfg.n_kv_head,
          f"{a}.attention.key_length": cfg.head_dim, f"{a}.attention.value_length": cfg.head_dim,
          f"{a}.rope.freq_base": Typed(T_F32, cfg.rope_theta),
          f"{a}.attention.layer_norm_rms_epsilon": Typed(T_F32, cfg.rms_eps),
          "tokenizer.ggml.model": "gpt2",
          "tokenizer.ggml.token_type": Typed(T_ARR, np.ones(4, np.int32), T_I32),
          "tokenizer.ggml.tokens": Typed(T_ARR, ["a", "b", "c", "d"], T_STR)}
    if arch == "qwen35":
        md.update({f"{a}.full_attention_interval": 4, f"{a}.ssm.time_step_rank": cfg.dn_num_v_heads,
                   f"{a}.ssm.group_count": cfg.dn_num_k_heads, f"{a}.ssm.state_size": cfg.dn_k_head_dim,
                   f"{a}.ssm.inner_size": cfg.dn_num_v_heads * cfg.dn_v_head_dim,
                   f"{a}.ssm.conv_kernel": cfg.dn_conv_kernel, f"{a}.rope.dimension_count": cfg.rope_dims})
    return md


def _bf16(w):
    """fp32 -> bf16 bytes, rounded to nearest even."""
    u = np.asarray(w, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).tobytes()


def build(path, cfg, seed, arch="qwen3", one_bit="blk.0.attn_k.weight", hadamard=0):
    """Write the GGUF; returns {name: (scales, codes)} of its ternary matrices as the file holds
    them (the 1-bit matrix as codes 0/2). hadamard: the block of a PrismML rotation declared in
    the metadata, with seeded signs for every projection input width (the weights stand for
    folded ones)."""
    specs = synth.small_model_tensors(cfg, seed, fp16_embedding=False)
    rng = np.random.default_rng(seed + 1)
    tensors, truth, k = [], {}, 0
    for sp in specs:
        name = sp.name
        if arch == "qwen35" and ".ffn_norm." in name:
            name = name.replace(".ffn_norm.", ".post_attention_norm.")
        if sp.kind == L.KIND_TERNARY:
            s = np.asarray(sp.scales, np.float16).reshape(-1)
            codes = sp.values.reshape(-1, 128)
            if name == one_bit:
                bits = rng.integers(0, 2, codes.shape, dtype=np.uint8)
                tid, raw, codes = Q.GGML_Q1_0, Q.q1_0_pack(s, bits), bits * 2
            else:
                tid = TERNARY_CYCLE[k % len(TERNARY_CYCLE)]
                k += 1
                raw = Q.ptq1_0_pack(s, codes) if tid == Q.GGML_PTQ1_0 else Q.q2_0_pack(s, codes)
            truth[name] = (sp.scales, codes.reshape(sp.rows, sp.cols))
            tensors.append((name, (sp.rows, sp.cols), tid, raw))
        elif sp.kind == L.KIND_Q8 and sp.role == L.ROLE_SSM_BETA:
            tensors.append((name, (sp.rows, sp.cols), Q.GGML_Q8_0,
                            Q.q8_0_pack(sp.scales.reshape(-1), sp.values.reshape(-1, 32))))
        elif sp.kind == L.KIND_Q8:
            w = sp.values.astype(np.float32) * np.repeat(sp.scales.astype(np.float32), 32, axis=1)
            tensors.append((name, (sp.rows, sp.cols), Q.GGML_BF16, _bf16(w)))
        else:
            v = np.asarray(sp.values, np.float32)
            shape = (v.shape[1],) if v.shape[0] == 1 else v.shape
            tensors.append((name, shape, Q.GGML_F32, v.tobytes()))
    # The embedding goes last: with an odd vocabulary its payload is not a multiple of the
    # alignment, and only the last tensor's size is exact from the offsets alone.
    tensors.sort(key=lambda t: t[0] == "token_embd.weight")
    md = _meta(cfg, arch)
    if hadamard:
        widths = input_widths(cfg)
        signs = np.concatenate([np.where(rng.random(w) < 0.5, -1, 1) for w in widths]).astype(np.int8)
        md.update({"prism.hadamard.block_size": hadamard,
                   "prism.hadamard.transform": "normalized-sylvester-walsh-hadamard",
                   "prism.hadamard.axis": "input-last-dimension",
                   "prism.hadamard.sign_widths": Typed(T_ARR, np.array(widths, np.int32), T_I32),
                   "prism.hadamard.sign_values": Typed(T_ARR, signs, T_I8)})
    write_gguf(path, md, tensors)
    return truth
