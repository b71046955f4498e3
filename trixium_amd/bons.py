"""BONS image writer and reader for the GPU host.

The writer lays quantized tensors out as row packets (trixium_amd.layout) and shards them by
output row over n_channels, adding the derived tensors a BONS image carries (the rope table,
the int16 companions of every F32 tensor and the int16 embedding table), as the reference writer
does (model/bons.py:342-459). The reader parses an image and hands back tensors
(model/bons.py:476-525); `entry_rows` returns a tensor's row packets in row order, the layout the
GPU keeps resident (one channel, rows back to back).
"""

import json
import math
from types import SimpleNamespace

import numpy as np

from . import layout as L
from .fixedpoint import fp16_split, scale_bias, result_shift, GS_MAX, GS_MAX_Q8


class TensorSpec:
    """One tensor to write. Ternary: scales (rows, cols/128) fp16 and codes (rows, cols) uint8 in
    {0,1,2} (w = code - 1); Q8: scales (rows, cols/32) and int8 values; F16/F32/NORM16: values.
    `loader`, in place of values, returns them when the writer reaches the tensor, so a converter
    holds one tensor's codes at a time (the reference's TensorSpec.loader, model/bons.py)."""

    def __init__(self, name, role, layer, kind, rows, cols, scales=None, values=None, flags=0,
                 bias=None, kseg=0, fixed_point=None, loader=None):
        self.name, self.role, self.layer, self.kind = name, role, layer, kind
        self.rows, self.cols, self.flags, self.kseg = rows, cols, flags, kseg
        self.scales, self.values, self.loader = scales, values, loader
        if values is not None and tuple(values.shape) != (rows, cols):
            raise ValueError(f"{name}: values {values.shape} != {(rows, cols)}")
        if kind in (L.KIND_TERNARY, L.KIND_TERNARY5, L.KIND_Q8):
            g = L.KIND_GROUP[kind]
            if scales is None or tuple(scales.shape) != (rows, cols // g):
                raise ValueError(f"{name}: scales must be (rows, cols/{g})")
            sc = np.asarray(scales, dtype=np.float16)
            self.bias = scale_bias(sc)
            self.rshift = result_shift(sc, self.bias, GS_MAX if kind != L.KIND_Q8 else GS_MAX_Q8)
            if fixed_point is not None:
                self.bias, self.rshift = fixed_point
        else:
            self.bias = (bias & 0xFF) if bias is not None else 0
            self.rshift = 0

    def load(self):
        """The values, from the loader when none are held."""
        if self.values is not None:
            return self.values
        v = self.loader()
        if tuple(v.shape) != (self.rows, self.cols):
            raise ValueError(f"{self.name}: loaded values {v.shape} != {(self.rows, self.cols)}")
        return v


def split_wide(spec, kseg_max=L.KSEG_MAX):
    """A ternary or Q8 matrix wider than kseg_max as K-segments (model/bons.py:83-115): nseg =
    ceil(cols / kseg_max) column ranges on whole scale groups (segment k ends at group
    floor(G k / nseg)), each flagged FLAG_KSEG with its index, named `<name>.k<k>`, and every one
    keeping the whole tensor's bias/rshift so the segment results add up. The token embedding
    stays whole (a lookup reads whole rows)."""
    if spec.kind == L.KIND_Q8:
        kseg_max = min(kseg_max, L.KSEG_MAX_Q8)
    if spec.kind not in (L.KIND_TERNARY, L.KIND_Q8) or spec.cols <= kseg_max or spec.role == L.ROLE_TOK_EMB:
        return [spec]
    g = L.KIND_GROUP[spec.kind]
    if kseg_max < g:
        raise ValueError(f"kseg_max {kseg_max} is narrower than the {g}-weight scale group")
    nseg, ngrp = -(-spec.cols // kseg_max), spec.cols // g
    edges = [ngrp * k // nseg * g for k in range(nseg + 1)]
    out = []
    for k in range(nseg):
        c0, c1 = edges[k], edges[k + 1]
        vals = None if spec.values is None else np.ascontiguousarray(spec.values[:, c0:c1])
        ld = None if spec.loader is None else (lambda c0=c0, c1=c1, f=spec.loader: np.ascontiguousarray(f()[:, c0:c1]))
        out.append(TensorSpec(f"{spec.name}.k{k}", spec.role, spec.layer, spec.kind, spec.rows, c1 - c0,
                              scales=np.ascontiguousarray(spec.scales[:, c0 // g:c1 // g]), values=vals,
                              flags=spec.flags | L.FLAG_KSEG, kseg=k, fixed_point=(spec.bias, spec.rshift),
                              loader=ld))
    return out


# Row-packet codecs -----------------------------------------------------------------------------

_POW3 = np.array([1, 3, 9, 27, 81], dtype=np.uint16)


def trit5_pack(codes):
    """(rows, cols) codes {0,1,2} -> (rows, 26*cols/128) bytes, base 3, lane 5i+k = digit k of
    byte i within every 128-group, lanes 128 and 129 zero."""
    rows, cols = codes.shape
    g = cols // L.GROUP
    c = np.asarray(codes, np.uint8).reshape(rows, g, 128)
    out = np.empty((rows, g, 26), np.uint8)
    d = c[:, :, :125].reshape(rows, g, 25, 5)
    out[:, :, :25] = d[..., 0] + 3 * d[..., 1] + 9 * d[..., 2] + 27 * d[..., 3] + 81 * d[..., 4]
    out[:, :, 25] = c[:, :, 125] + 3 * c[:, :, 126] + 9 * c[:, :, 127]
    return out.reshape(rows, g * 26)


def trit5_unpack(body, cols):
    rows = body.shape[0]
    g = cols // L.GROUP
    b = body[:, :26 * g].astype(np.uint16).reshape(rows, g, 26, 1)
    digits = (b // _POW3) % 3
    return digits.reshape(rows, g, 130)[:, :, :128].reshape(rows, cols).astype(np.uint8)


def pack2(codes):
    """(rows, cols) codes -> (rows, cols/4) bytes, code j at bits 2*(j%4) of byte j//4."""
    rows, cols = codes.shape
    c = codes.astype(np.uint8).reshape(rows, cols // 4, 4)
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).astype(np.uint8)


def unpack2(body, cols):
    b = body[:, :cols // 4]
    return np.stack([(b >> (2 * k)) & 3 for k in range(4)], axis=-1).reshape(b.shape[0], cols).astype(np.uint8)


def encode_rows(kind, cols, scales, values):
    """Row packets of `values` (and `scales`) -> (rows, row_bytes) uint8."""
    rows = values.shape[0]
    out = np.zeros((rows, L.row_bytes(cols, kind)), dtype=np.uint8)
    off = L.scale_beats(cols, kind) * L.BEAT
    if kind in L.KIND_GROUP:
        sb = np.ascontiguousarray(np.asarray(scales, dtype=np.float16)).view(np.uint8).reshape(rows, -1)
        out[:, :sb.shape[1]] = sb
    if kind == L.KIND_TERNARY:
        body = pack2(values)
    elif kind == L.KIND_TERNARY5:
        body = trit5_pack(values)
    elif kind == L.KIND_Q8:
        body = np.ascontiguousarray(values.astype(np.int8)).view(np.uint8)
    elif kind == L.KIND_F16:
        body = np.ascontiguousarray(values.astype(np.float16)).view(np.uint8).reshape(rows, -1)
    elif kind == L.KIND_F32:
        body = np.ascontiguousarray(values.astype(np.float32)).view(np.uint8).reshape(rows, -1)
    elif kind == L.KIND_NORM16:
        body = np.ascontiguousarray(values.astype("<i2")).view(np.uint8).reshape(rows, -1)
    else:
        raise ValueError(f"kind {kind}")
    out[:, off:off + body.shape[1]] = body
    return out


def decode_rows(kind, cols, packets):
    """(rows, row_bytes) packets -> (scales or None, values)."""
    data = np.asarray(packets, dtype=np.uint8).reshape(-1, L.row_bytes(cols, kind))
    rows = data.shape[0]
    scales = None
    if kind in L.KIND_GROUP:
        scales = np.ascontiguousarray(data[:, :2 * (cols // L.KIND_GROUP[kind])]).view(np.float16)
    body = np.ascontiguousarray(data[:, L.scale_beats(cols, kind) * L.BEAT:])
    if kind == L.KIND_TERNARY:
        values = unpack2(body, cols)
    elif kind == L.KIND_TERNARY5:
        values = trit5_unpack(body, cols)
    elif kind == L.KIND_Q8:
        values = body[:, :cols].copy().view(np.int8)
    elif kind == L.KIND_F16:
        values = body[:, :2 * cols].copy().view(np.float16)
    elif kind == L.KIND_F32:
        values = body[:, :4 * cols].copy().view(np.float32)
    elif kind == L.KIND_NORM16:
        values = body[:, :2 * cols].copy().view(np.int16)
    else:
        raise ValueError(f"kind {kind}")
    return scales, values.reshape(rows, cols)


# Derived tensors -------------------------------------------------------------------------------

def rope_tables(cfg, positions):
    """cos/sin (len(positions), rope_dims/2) in float64 with the YaRN ramp of llama.cpp's
    rope_yarn when cfg.yarn_factor != 1 (the rule of model/golden.py:189-213)."""
    n = cfg.rope_dims or cfg.head_dim
    p = np.asarray(positions, dtype=np.float64)[:, None]
    d = np.arange(n // 2, dtype=np.float64)[None, :]
    extrap = p * np.power(float(cfg.rope_theta), -2.0 * d / n)
    fs = 1.0 / cfg.yarn_factor
    interp = fs * extrap
    mscale = 1.0
    if cfg.yarn_factor != 1.0:
        def corr(rot):
            return n * math.log(cfg.yarn_orig_ctx / (rot * 2 * math.pi)) / (2 * math.log(cfg.rope_theta))
        lo = max(0.0, math.floor(corr(32.0)))
        hi = min(n - 1.0, math.ceil(corr(1.0)))
        ramp = 1.0 - np.clip((d - lo) / max(0.001, hi - lo), 0.0, 1.0)
        theta = interp * (1 - ramp) + extrap * ramp
        mscale = 1.0 + 0.1 * math.log(1.0 / fs)
    else:
        theta = interp
    return np.cos(theta) * mscale, np.sin(theta) * mscale


def rope_q14(cfg, n_pos):
    """The image's rope table: one row per position, [cos | sin] of rope_tables in Q14 int16
    (model/bons.py:356-367; Q14 holds YaRN's mscale > 1)."""
    cos, sin = rope_tables(cfg, np.arange(n_pos))
    tab = np.concatenate([cos, sin], axis=1)
    return np.clip(np.round(tab * (1 << 14)), -32767, 32767).astype(np.int16)


def image_rope_table(img):
    """The image's Q14 rope table (int16 [max_ctx, rope_dims]) when it differs from plain RoPE
    (theta^(-2i/n), no YaRN: what model/fastref.py computes), else None. A YaRN-scaled model
    exists only in this table (the header has no YaRN fields); the firmware and the mirror read
    it per position (model/mirror.py:478-483)."""
    e = img.find(L.ROLE_ROPE_TAB, 0)
    if e is None:
        return None
    _, t14 = img.entry_tensor(e)
    t14 = np.asarray(t14, dtype=np.int16).reshape(e["rows"], e["cols"])
    h = img.header
    plain = type("PlainRope", (), dict(rope_dims=h["rope_dims"], head_dim=h["head_dim"],
                                       rope_theta=float(h["rope_theta"]), yarn_factor=1.0,
                                       yarn_orig_ctx=0))
    return None if np.array_equal(t14, rope_q14(plain, e["rows"])) else t14


def embed_bfp_rows(codes, scales):
    """Ternary embedding rows -> the int16 BFP table (mantissas (rows, cols) int16, exponents
    (rows,) int32), integer-exact: every group's (code-1)*m11 aligned to the row's smallest scale
    exponent (alignment capped at 20 bits), the row's largest aligned |m11| over groups with a
    nonzero code normalised into [2**14, 2**15), then truncated to int16
    (the contract of model/bons.py:204-236)."""
    m11, e16 = fp16_split(scales)
    rows, cols = codes.shape
    g = cols // L.GROUP
    c = np.asarray(codes, np.uint8).reshape(rows, g, L.GROUP)
    emin = e16.min(axis=1, keepdims=True)
    sh = np.minimum(e16 - emin, 20)
    live = (c != 1).any(axis=2)
    amax = np.where(live, np.abs(m11) << sh, 0).max(axis=1)
    blen = np.array([int(a).bit_length() for a in amax], dtype=np.int64)
    k2 = blen - 15
    net = sh - k2[:, None]
    # A group's mantissas take three values, (code - 1) * m11 shifted by the group's net exponent
    # (an arithmetic right shift rounds the negative one down): gather them per code.
    # A group's mantissas are (code - 1) * pos, pos = m11 shifted by the group's net exponent,
    # except that an arithmetic right shift of -m11 rounds down: one less when bits drop out.
    m = m11.astype(np.int64)
    up, down = np.maximum(net, 0), np.maximum(-net, 0)
    pos = np.where(net >= 0, m << up, m >> down).astype(np.int16)
    low = (np.where(net >= 0, 0, m & ((np.int64(1) << down) - 1)) != 0).astype(np.int16)
    mant = np.empty((rows, g, L.GROUP), np.int16)
    for r in range(0, rows, 8192):
        q = c[r:r + 8192].astype(np.int16) - 1
        blk = q * pos[r:r + 8192, :, None]
        if low[r:r + 8192].any():
            blk -= (q < 0).view(np.int8).astype(np.int16) * low[r:r + 8192, :, None]
        mant[r:r + 8192] = blk
    return mant.reshape(rows, cols), (emin[:, 0] + k2).astype(np.int32)


def float_bfp_rows(values):
    """Float embedding rows -> int16 BFP rows: per row the exponent puts |max| in
    [2**14, 2**15), mantissas rounded half to even and clipped to +-32767."""
    v = np.asarray(values, dtype=np.float64)
    amax = np.abs(v).max(axis=1)
    e = np.where(amax > 0, np.floor(np.log2(np.maximum(amax, 1e-300))).astype(np.int64) - 14, 0)
    mant = np.clip(np.round(v * np.exp2(-e)[:, None]), -32767, 32767)
    return mant.astype(np.int16), e.astype(np.int32)


def emb16_specs(mant, exps):
    rows, cols = mant.shape
    erows = L.cdiv(rows, 16)
    etab = np.zeros((erows, 16), dtype=np.int16)
    etab.reshape(-1)[:rows] = exps.astype(np.int16)
    return [TensorSpec("token_embd.bfp16", L.ROLE_TOK_EMB16, 0, L.KIND_NORM16, rows, cols, values=mant),
            TensorSpec("token_embd.bfp16_exp", L.ROLE_TOK_EMB16_EXP, 0, L.KIND_NORM16, erows, 16,
                       values=etab, flags=L.FLAG_REPLICATED)]


# Writer ----------------------------------------------------------------------------------------

def write_image(cfg, tensors, n_channels, path, tokenizer_sha256=b"", manifest_path=None,
                emb16=True, trit5=False):
    """Write a BONS v3 image; returns the manifest dict (model/bons.py:342-459's contract:
    derived rope table, .w16 companions, int16 embedding table, optional trit5 storage)."""
    tensors = list(tensors)
    if cfg.max_ctx and cfg.head_dim:
        t14 = rope_q14(cfg, cfg.max_ctx)
        tensors.append(TensorSpec("rope_tab", L.ROLE_ROPE_TAB, 0, L.KIND_NORM16, cfg.max_ctx,
                                  t14.shape[1], values=t14, flags=L.FLAG_REPLICATED))
    for spec in [t for t in tensors if t.kind == L.KIND_F32]:
        w = spec.values.astype(np.float64)
        e = L.norm16_exp(w)
        q = np.round(w * 2.0**(-e))
        tensors.append(TensorSpec(spec.name.replace(".weight", "") + ".w16", spec.role, spec.layer,
                                  L.KIND_NORM16, spec.rows, spec.cols, values=q.astype(np.int16),
                                  flags=spec.flags, bias=e))
    emb = [t for t in tensors if t.role == L.ROLE_TOK_EMB and t.kind == L.KIND_TERNARY]
    if emb16 and emb and not any(t.role == L.ROLE_TOK_EMB16 for t in tensors):
        if cfg.hadamard_block:
            # A rotated table is restored to the plain basis here, in row blocks.
            from .hadamard import restored_bfp_rows
            codes, sig = emb[0].load(), cfg.hadamard_signs[emb[0].cols]
            parts = [restored_bfp_rows(emb[0].scales[r:r + 8192], codes[r:r + 8192], sig, cfg.hadamard_block)
                     for r in range(0, emb[0].rows, 8192)]
            tensors.extend(emb16_specs(np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])))
        else:
            tensors.extend(emb16_specs(*embed_bfp_rows(emb[0].load(), emb[0].scales)))
    if trit5:
        has16 = any(t.role == L.ROLE_TOK_EMB16 for t in tensors)
        for spec in tensors:
            if spec.kind == L.KIND_TERNARY and (spec.role in L.TRIT5_ROLES or
                                                (spec.role == L.ROLE_TOK_EMB and has16)):
                spec.kind = L.KIND_TERNARY5

    per_chan = []
    base = 0
    for spec in tensors:
        nrows = spec.rows if spec.flags & L.FLAG_REPLICATED else L.shard_rows(spec.rows, n_channels, 0)[1]
        n = nrows * L.row_beats(spec.cols, spec.kind)
        per_chan.append((base, n))
        base += n
    payload_beats = base
    table_pad = L.cdiv(len(tensors) * L.ENTRY_SIZE, L.HEADER_SIZE) * L.HEADER_SIZE
    payload_off = L.HEADER_SIZE + table_pad
    chan_bytes = payload_beats * L.BEAT
    image = np.zeros(payload_off + n_channels * chan_bytes, dtype=np.uint8)
    entries, man = [], []
    for spec, (b0, nb) in zip(tensors, per_chan):
        packets = encode_rows(spec.kind, spec.cols, spec.scales, spec.load())
        crc = 0
        for c in range(n_channels):
            r0, nr = (0, spec.rows) if spec.flags & L.FLAG_REPLICATED else L.shard_rows(spec.rows, n_channels, c)
            chunk = packets[r0:r0 + nr].reshape(-1)
            crc = L.crc32(chunk, crc)
            at = payload_off + c * chan_bytes + b0 * L.BEAT
            image[at:at + chunk.size] = chunk
        entries.append(L.pack_entry(spec.role, spec.kind, spec.flags, spec.layer, spec.rows,
                                    spec.cols, b0, nb, crc, spec.bias, spec.rshift, spec.name,
                                    kseg=spec.kseg))
        man.append({"name": spec.name, "role": L.ROLE_NAMES[spec.role], "layer": spec.layer,
                    "kind": L.KIND_NAMES[spec.kind], "flags": spec.flags, "rows": spec.rows,
                    "cols": spec.cols, "chan_base_beats": b0, "chan_len_beats": nb, "crc32": crc,
                    "bias": spec.bias, "rshift": spec.rshift})
    table = b"".join(entries)
    tcrc = L.crc32(table)
    image[:L.HEADER_SIZE] = np.frombuffer(L.pack_header(cfg, n_channels, len(tensors),
                                                         payload_beats, tcrc, tokenizer_sha256), np.uint8)
    image[L.HEADER_SIZE:L.HEADER_SIZE + len(table)] = np.frombuffer(table, np.uint8)
    image.tofile(path)
    manifest = {"model": cfg.name, "n_channels": n_channels, "payload_beats": payload_beats,
                "payload_bytes_per_channel": chan_bytes, "table_crc32": tcrc, "tensors": man}
    if manifest_path is not None:
        with open(manifest_path, "w", encoding="utf-8") as f:
            json.dump(manifest, f, indent=2)
    return manifest


# Reader ----------------------------------------------------------------------------------------

class _Names(dict):
    """name -> entry; a lookup by a name longer than the 24-byte field finds its truncation."""

    def __missing__(self, name):
        e = dict.get(self, name[:L.NAME_BYTES])
        if e is None:
            raise KeyError(name)
        return e


class BONSReader:
    def __init__(self, path):
        self.data = np.memmap(path, dtype=np.uint8, mode="r")
        if len(self.data) < L.HEADER_SIZE:
            raise ValueError("file too short for a BONS header")
        self.header = L.unpack_header(self.data[:L.HEADER_SIZE])
        off = self.header["table_offset"]
        self.entries = [L.unpack_entry(self.data[off + i * L.ENTRY_SIZE: off + (i + 1) * L.ENTRY_SIZE])
                        for i in range(self.header["n_tensors"])]
        self.by_name = _Names()
        for e in self.entries:
            self.by_name.setdefault(e["name"], e)

    def channel_payload(self, channel):
        h = self.header
        n = h["payload_beats"] * L.BEAT
        start = h["payload_offset"] + channel * n
        return self.data[start:start + n]

    def entry_channel_bytes(self, e, channel):
        ch = self.channel_payload(channel)
        return ch[e["chan_base_beats"] * L.BEAT:(e["chan_base_beats"] + e["chan_len_beats"]) * L.BEAT]

    def tensor_channel_bytes(self, name, channel):
        return self.entry_channel_bytes(self.by_name[name], channel)

    def entry_rows(self, e):
        """All row packets of an entry in row order: (rows, row_bytes) uint8."""
        rb = L.row_bytes(e["cols"], e["kind"])
        if e["flags"] & L.FLAG_REPLICATED or self.header["n_channels"] == 1:
            return np.asarray(self.entry_channel_bytes(e, 0)).reshape(-1, rb)
        return np.concatenate([np.asarray(self.entry_channel_bytes(e, c)).reshape(-1, rb)
                               for c in range(self.header["n_channels"])], axis=0)

    def entry_tensor(self, e):
        return decode_rows(e["kind"], e["cols"], self.entry_rows(e))

    def tensor(self, name):
        return self.entry_tensor(self.by_name[name])

    def find(self, role, layer=0, kind=None):
        """First entry of (role, layer[, kind]); the firmware's lookup key (names collide)."""
        for e in self.entries:
            if e["role"] == role and e["layer"] == layer and (kind is None or e["kind"] == kind):
                return e
        return None

    def ksegs(self, e):
        """The K-segments of a split entry in order (model/fastref.py:96-101), else [e]."""
        if not e["flags"] & L.FLAG_KSEG:
            return [e]
        segs = [t for t in self.entries if t["role"] == e["role"] and t["layer"] == e["layer"]
                and t["kind"] == e["kind"] and t["flags"] & L.FLAG_KSEG]
        return sorted(segs, key=lambda t: t["kseg"])
