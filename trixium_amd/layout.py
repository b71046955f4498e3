"""BONS weight-image layout contract, as the GPU host code reads and writes it.

The on-disk format is fixed by the reference (model/layout.py:39-121 kinds/roles/flags,
model/layout.py:184-223 row-packet geometry, model/layout.py:233-333 header and entry structs);
this module states the same byte layout independently so that images written by either side
load on the other.

Row packet of a quantized tensor row (model/layout.py:17-30):
    [ceil(G/16) beats of fp16 group scales][code beats]       one beat = 32 bytes
    2-bit  (KIND_TERNARY):  G beats, code j of the row at byte j//4, bits 2*(j%4)
    trit5  (KIND_TERNARY5): 26 bytes per 128-group, byte i of a group holds the base-3
                            digits of lanes 5i..5i+4 (lane 5i+k is digit k; lanes 128/129
                            are zero), the code area padded to a whole beat.
"""

import struct
import zlib

BEAT = 32                  # bytes per beat
GROUP = 128                # ternary weights per fp16 scale
GROUP_Q8 = 32              # int8 weights per fp16 scale
SCALES_PER_BEAT = BEAT // 2
TRIT5_GROUP_BYTES = 26     # ceil(128 / 5)

# Tensor kinds (model/layout.py:45-54).
KIND_TERNARY, KIND_Q8, KIND_F16, KIND_F32, KIND_NORM16, KIND_TERNARY5 = 0, 1, 2, 3, 4, 5
KIND_NAMES = {KIND_TERNARY: "ternary", KIND_Q8: "q8", KIND_F16: "f16", KIND_F32: "f32",
              KIND_NORM16: "norm16", KIND_TERNARY5: "ternary5"}
KIND_GROUP = {KIND_TERNARY: GROUP, KIND_TERNARY5: GROUP, KIND_Q8: GROUP_Q8}

# Tensor flags (model/layout.py:84-92).
FLAG_REPLICATED = 0x01
FLAG_KSEG = 0x02
KSEG_MAX = 16384
KSEG_MAX_Q8 = 255 * 32      # a Q8 segment: at most 255 code beats of 32 columns

# Tensor roles (model/layout.py:95-115).
ROLE_TOK_EMB, ROLE_OUT_NORM, ROLE_LM_HEAD = 0, 1, 2
ROLE_ATTN_NORM, ROLE_ATTN_Q, ROLE_ATTN_K, ROLE_ATTN_V, ROLE_ATTN_OUT = 3, 4, 5, 6, 7
ROLE_ATTN_Q_NORM, ROLE_ATTN_K_NORM = 8, 9
ROLE_FFN_NORM, ROLE_FFN_GATE, ROLE_FFN_UP, ROLE_FFN_DOWN = 10, 11, 12, 13
ROLE_ROPE_TAB, ROLE_TOK_EMB16, ROLE_TOK_EMB16_EXP = 14, 15, 16
ROLE_ATTN_QKV, ROLE_ATTN_ZGATE, ROLE_SSM_OUT, ROLE_SSM_BETA, ROLE_SSM_ALPHA = 17, 18, 19, 20, 21
ROLE_SSM_CONV, ROLE_SSM_A, ROLE_SSM_DT, ROLE_SSM_NORM, ROLE_HADAMARD = 22, 23, 24, 25, 26

def hadamard_layer(width_index, block_index):
    """The entry `layer` of a rotation block tensor: width index * 256 + block (model/layout.py:124-128)."""
    if not (0 <= width_index < 4 and 0 <= block_index < 256):
        raise ValueError("rotation block out of range")
    return width_index * 256 + block_index


# Roles whose ternary weights the writer stores as trit5 when asked (model/layout.py:131-133).
TRIT5_ROLES = (ROLE_ATTN_Q, ROLE_ATTN_K, ROLE_ATTN_V, ROLE_ATTN_OUT, ROLE_FFN_GATE,
               ROLE_FFN_UP, ROLE_FFN_DOWN, ROLE_LM_HEAD, ROLE_ATTN_QKV, ROLE_ATTN_ZGATE,
               ROLE_SSM_OUT)

ROLE_NAMES = {
    0: "tok_emb", 1: "out_norm", 2: "lm_head", 3: "attn_norm", 4: "attn_q", 5: "attn_k",
    6: "attn_v", 7: "attn_out", 8: "attn_q_norm", 9: "attn_k_norm", 10: "ffn_norm",
    11: "ffn_gate", 12: "ffn_up", 13: "ffn_down", 14: "rope_tab", 15: "tok_emb16",
    16: "tok_emb16_exp", 17: "attn_qkv", 18: "attn_zgate", 19: "ssm_out", 20: "ssm_beta",
    21: "ssm_alpha", 22: "ssm_conv", 23: "ssm_a", 24: "ssm_dt", 25: "ssm_norm",
    26: "hadamard",
}


def is_ternary(kind):
    return kind == KIND_TERNARY or kind == KIND_TERNARY5


def cdiv(a, b):
    return -(-a // b)


def groups(cols, kind):
    g = KIND_GROUP[kind]
    if cols % g:
        raise ValueError(f"{cols} columns are not a multiple of the {g}-wide group")
    return cols // g


def scale_beats(cols, kind):
    """Beats of fp16 scales at the head of every row (0 for unscaled kinds)."""
    if kind in KIND_GROUP:
        return cdiv(groups(cols, kind), SCALES_PER_BEAT)
    return 0


def code_beats(cols, kind):
    """Code beats per row as the engine counts them (one per ternary 128-group)."""
    if is_ternary(kind):
        return groups(cols, kind)
    if kind == KIND_Q8:
        return groups(cols, kind)
    width = {KIND_F16: 2, KIND_F32: 4, KIND_NORM16: 2}[kind]
    return cdiv(width * cols, BEAT)


def mem_code_beats(cols, kind):
    """Code beats per row in memory (trit5 packs a group into 26 bytes)."""
    if kind == KIND_TERNARY5:
        return cdiv(TRIT5_GROUP_BYTES * groups(cols, kind), BEAT)
    return code_beats(cols, kind)


def row_beats(cols, kind):
    return scale_beats(cols, kind) + mem_code_beats(cols, kind)


def row_bytes(cols, kind):
    return BEAT * row_beats(cols, kind)


def shard_rows(rows, n_channels, channel):
    if rows % n_channels:
        raise ValueError(f"{rows} rows do not divide over {n_channels} channels")
    per = rows // n_channels
    return channel * per, per


def norm16_exp(values):
    """Exponent of a NORM16 companion: smallest e with |v| * 2^-e <= 32767
    (model/layout.py:56-63)."""
    import math
    import numpy as np
    a = float(np.abs(values).max()) if values.size else 0.0
    if a == 0.0:
        return -13
    return math.ceil(math.log2(a / 32767.0))


# Header and table entries (model/layout.py:233-333) ---------------------------------------------

MAGIC = 0x534E4F42          # "BONS"
VERSION = 3
VERSIONS_READ = (2, 3)
HEADER_SIZE = 4096
ENTRY_SIZE = 64
NAME_BYTES = 24
HYB_EMB16_RESTORED = 0x01

_HDR_KEYS = ("magic", "version", "n_layer", "n_embd", "n_head", "n_kv_head", "head_dim",
             "ffn_dim", "vocab", "rope_theta", "rms_eps", "max_ctx", "n_channels",
             "n_tensors", "table_offset", "payload_offset", "payload_beats", "mode",
             "table_crc32", "tokenizer_sha256")
_HYB = struct.Struct("<2Q7H2B4I")            # offsets 112..159
_HYB_OFF = 112
_ENTRY = struct.Struct("<4B2H2I2QI2B2x24s")


def _pack_header_fields(vals):
    # vals are in _HDR_KEYS order; the u64 payload_beats at offset 64 sits between u32 fields,
    # so the struct is assembled field by field to keep the offsets of the contract.
    out = bytearray(112)
    u32 = lambda off, v: struct.pack_into("<I", out, off, v & 0xFFFFFFFF)
    u32(0, vals[0]); u32(4, vals[1]); u32(8, vals[2]); u32(12, vals[3]); u32(16, vals[4])
    u32(20, vals[5]); u32(24, vals[6]); u32(28, vals[7]); u32(32, vals[8]); u32(36, vals[9])
    struct.pack_into("<f", out, 40, vals[10])
    u32(44, vals[11]); u32(48, vals[12]); u32(52, vals[13]); u32(56, vals[14]); u32(60, vals[15])
    struct.pack_into("<Q", out, 64, vals[16])
    u32(72, vals[17]); u32(76, vals[18])
    out[80:112] = vals[19][:32].ljust(32, b"\x00")
    return bytes(out)


def pack_header(cfg, n_channels, n_tensors, payload_beats, table_crc32, tokenizer_sha256=b""):
    table_bytes = cdiv(n_tensors * ENTRY_SIZE, HEADER_SIZE) * HEADER_SIZE
    base = _pack_header_fields((
        MAGIC, VERSION, cfg.n_layer, cfg.n_embd, cfg.n_head, cfg.n_kv_head, cfg.head_dim,
        cfg.ffn_dim, cfg.vocab, int(cfg.rope_theta), cfg.rms_eps, cfg.max_ctx, n_channels,
        n_tensors, HEADER_SIZE, HEADER_SIZE + table_bytes, payload_beats, 0, table_crc32,
        tokenizer_sha256))
    ltypes = 0
    for l in range(cfg.n_layer):
        if cfg.layer_type(l) == "deltanet":
            ltypes |= 1 << l
    widths = sorted(cfg.hadamard_signs) if cfg.hadamard_signs else []
    if len(widths) > 4:
        raise ValueError("at most four Hadamard widths fit the header")
    hyb = _HYB.pack(ltypes & (2**64 - 1), ltypes >> 64, cfg.dn_num_v_heads, cfg.dn_num_k_heads,
                    cfg.dn_k_head_dim, cfg.dn_v_head_dim, cfg.dn_conv_kernel, cfg.rope_dims,
                    cfg.hadamard_block, int(bool(cfg.attn_gated)),
                    HYB_EMB16_RESTORED if cfg.hadamard_block else 0, *(widths + [0] * (4 - len(widths))))
    return (base + hyb).ljust(HEADER_SIZE, b"\x00")


def unpack_header(data):
    data = bytes(data[:HEADER_SIZE])
    u32 = lambda off: struct.unpack_from("<I", data, off)[0]
    vals = [u32(4 * i) for i in range(10)] + [struct.unpack_from("<f", data, 40)[0]]
    vals += [u32(44), u32(48), u32(52), u32(56), u32(60), struct.unpack_from("<Q", data, 64)[0],
             u32(72), u32(76), data[80:112]]
    h = dict(zip(_HDR_KEYS, vals))
    if h["magic"] != MAGIC:
        raise ValueError("not a BONS image")
    if h["version"] not in VERSIONS_READ:
        raise ValueError(f"BONS version {h['version']} is not supported")
    hyb = _HYB.unpack_from(data, _HYB_OFF) if h["version"] >= 3 else (0,) * 15
    lt = hyb[0] | (hyb[1] << 64)
    h["layer_types"] = tuple("deltanet" if (lt >> l) & 1 else "attn" for l in range(h["n_layer"]))
    (h["dn_num_v_heads"], h["dn_num_k_heads"], h["dn_k_head_dim"], h["dn_v_head_dim"],
     h["dn_conv_kernel"], h["rope_dims"], h["hadamard_block"]) = hyb[2:9]
    h["attn_gated"], h["hyb_flags"] = hyb[9], hyb[10]
    h["hadamard_widths"] = tuple(w for w in hyb[11:15] if w)
    return h


def pack_entry(role, kind, flags, layer, rows, cols, chan_base_beats, chan_len_beats, crc32,
               bias=0, rshift=0, name="", kseg=0):
    return _ENTRY.pack(role, kind, flags, kseg, layer, KIND_GROUP.get(kind, 0), rows, cols,
                       chan_base_beats, chan_len_beats, crc32, bias & 0xFF, rshift & 0xFF,
                       name.encode()[:NAME_BYTES])


def unpack_entry(data, offset=0):
    f = _ENTRY.unpack_from(bytes(data), offset)
    return {"role": f[0], "kind": f[1], "flags": f[2], "kseg": f[3], "layer": f[4],
            "group": f[5], "rows": f[6], "cols": f[7], "chan_base_beats": f[8],
            "chan_len_beats": f[9], "crc32": f[10], "bias": f[11], "rshift": f[12],
            "name": f[13].rstrip(b"\x00").decode(errors="replace")}


def crc32(data, start=0):
    return zlib.crc32(bytes(data), start) & 0xFFFFFFFF
