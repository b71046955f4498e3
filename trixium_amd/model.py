"""Batch-1 greedy decoder on the GPU (host side of the trx_model_* entry points).

`Decoder` holds one BONS model resident in HBM and runs the token loop of the HIP library: one
position per forward, the argmax on the device, every per-token launch replayed from one captured
hipGraph. Its methods mirror model/golden.py:FloatModel (reset / forward / generate,
golden.py:304-320,436-470); the arithmetic is model/fastref.py:HybridRef's (fp32 activations,
ternary weights, fp16 KV cache on the GPU).

Differences from FloatModel, both from the firmware's loop (model/mirror.py:1036-1044,
firmware/infer.c:2001): `generate` runs no forward after its last output token, so the position
afterwards is len(prompt) + n - 1; and the logits are computed only where the caller asks for
them (the last fed position), not at every prefill position.
"""

import ctypes

import numpy as np

from . import _lib
from . import layout as L
from .configs import ModelConfig
from .hadamard import image_rotation

f32 = np.float32

(READ_LOGITS, READ_HIDDEN, READ_POSITION, READ_TOKEN, READ_OUT, READ_SLOT, READ_QKV, READ_ATTN, READ_ACT,
 READ_RESIDUAL) = range(10)
(INFO_ARENA_BYTES, INFO_DEVICE_BYTES, INFO_STREAM, INFO_WEIGHT_BYTES, _INFO_UNUSED, INFO_PACKED_OPS, INFO_ATTN_SPLITS,
 INFO_ATTN_PASS, INFO_TABLE_FREE_OPS, INFO_KV_PIN) = range(10)

# Projections run by the packed GEMV (TRX_PACK_* bits; PACK_AUTO lets the library choose).
PACK_QKV, PACK_O, PACK_GATE_UP, PACK_DOWN, PACK_HEAD, PACK_DN = 1, 2, 4, 8, 16, 32
PACK_ALL, PACK_AUTO = 63, -1
CKPT_SAVE, CKPT_RESTORE = 0, 1

# Ranges of the counter-based synthetic weights (the ternary group scales and the RMSNorm gains).
SYNTH_SCALE = (0.01, 0.05)
SYNTH_GAIN = (0.8, 1.2)

_LAYER_MATRICES_ATTN = (L.ROLE_ATTN_Q, L.ROLE_ATTN_K, L.ROLE_ATTN_V, L.ROLE_ATTN_OUT)
_LAYER_MATRICES_DN = (L.ROLE_ATTN_QKV, L.ROLE_ATTN_ZGATE, L.ROLE_SSM_OUT)
_LAYER_MATRICES_FFN = (L.ROLE_FFN_GATE, L.ROLE_FFN_UP, L.ROLE_FFN_DOWN)


def rope_frequencies(theta, rope_n):
    """theta**(-2i/n) evaluated in float32 (model/fastref.py:62-63)."""
    return np.array([f32(f32(theta) ** f32(-2.0 * i / rope_n)) for i in range(rope_n // 2)], dtype=f32)


def layer_type_bits(layer_types, n_layer):
    bits = 0
    for l in range(n_layer):
        if layer_types and layer_types[l] == "deltanet":
            bits |= 1 << l
    return (bits & (2**64 - 1), bits >> 64)


def make_config(mc, weight_kind, head_kind, head_tied, emb_mode, emb_kind, max_ctx=None, max_new=256,
                packed_ops=PACK_AUTO, prefill_chunk=0, table_free_ops=PACK_AUTO):
    """trx_model_config from a ModelConfig (or a BONS header turned into one)."""
    c = _lib.ModelConfig()
    for name in ("n_layer", "n_embd", "n_head", "n_kv_head", "head_dim", "ffn_dim", "vocab",
                 "rope_dims", "dn_num_v_heads", "dn_num_k_heads", "dn_k_head_dim", "dn_v_head_dim",
                 "dn_conv_kernel"):
        setattr(c, name, int(getattr(mc, name)))
    c.max_ctx = int(max_ctx or mc.max_ctx)
    c.rms_eps = float(mc.rms_eps)
    c.attn_gated = int(bool(mc.attn_gated))
    lo, hi = layer_type_bits(mc.layer_types, mc.n_layer)
    c.layer_types[0], c.layer_types[1] = lo, hi
    c.weight_kind, c.head_kind, c.head_tied = weight_kind, head_kind, int(bool(head_tied))
    c.emb_mode, c.emb_kind, c.max_new = emb_mode, emb_kind, int(max_new)
    c.packed_ops = int(packed_ops)
    c.prefill_chunk = int(prefill_chunk)
    c.table_free_ops = int(table_free_ops)
    return c


def config_from_header(h, name="bons-image"):
    return ModelConfig(name=name, n_layer=h["n_layer"], n_embd=h["n_embd"], n_head=h["n_head"],
                       n_kv_head=h["n_kv_head"], head_dim=h["head_dim"], ffn_dim=h["ffn_dim"],
                       vocab=h["vocab"], rope_theta=float(h["rope_theta"]), rms_eps=float(h["rms_eps"]),
                       max_ctx=h["max_ctx"], layer_types=tuple(h["layer_types"]),
                       dn_num_v_heads=h["dn_num_v_heads"], dn_num_k_heads=h["dn_num_k_heads"],
                       dn_k_head_dim=h["dn_k_head_dim"], dn_v_head_dim=h["dn_v_head_dim"],
                       dn_conv_kernel=h["dn_conv_kernel"], rope_dims=h["rope_dims"],
                       attn_gated=bool(h["attn_gated"]))


class Decoder:
    """One model resident on the GPU and its decode state."""

    def __init__(self, mc, cfg, use_graph=True):
        self.mc = mc
        self.cfg = cfg
        self.vocab, self.n_embd = cfg.vocab, cfg.n_embd
        self.use_graph = use_graph
        rope_n = mc.rope_dims or mc.head_dim
        self.rope_freq = rope_frequencies(mc.rope_theta, rope_n)
        h = ctypes.c_void_p()
        _lib.call("trx_model_create", ctypes.byref(cfg),
                  self.rope_freq.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), ctypes.byref(h))
        self._h = h.value

    # Construction ------------------------------------------------------------------------------
    @classmethod
    def from_image(cls, img, max_ctx=None, max_new=256, use_graph=True, packed_ops=PACK_AUTO, prefill_chunk=0,
                   table_free_ops=PACK_AUTO):
        """Load a BONS image (path or BONSReader) into HBM. prefill_chunk > 0: forward() and
        generate() run all but the last fed token through the batched prefill, that many
        positions per weight pass (0: one position per forward, as the firmware's loop)."""
        from .bons import BONSReader
        if isinstance(img, str):
            img = BONSReader(img)
        mc = config_from_header(img.header)
        nl = mc.n_layer
        kinds = {img.find(r, l)["kind"] for l in range(nl)
                 for r in ((_LAYER_MATRICES_DN if mc.layer_type(l) == "deltanet" else _LAYER_MATRICES_ATTN)
                           + _LAYER_MATRICES_FFN)}
        if len(kinds) != 1 or not L.is_ternary(next(iter(kinds))):
            raise ValueError(f"layer matrices must share one ternary kind, found {sorted(kinds)}")
        weight_kind = kinds.pop()
        head = img.find(L.ROLE_LM_HEAD, 0)
        emb = img.find(L.ROLE_TOK_EMB, 0)
        rot = image_rotation(img)
        emb_mode = 0
        if img.find(L.ROLE_TOK_EMB16, 0) is None:
            # Without the int16 table, a rotated image's rows are restored to the plain basis in
            # integers per token (the firmware's embed_row_restore, model/bons.py:262-295).
            if rot is None or emb is None or not L.is_ternary(emb["kind"]) or mc.n_embd not in rot[2]:
                raise ValueError("the image has no int16 embedding table (token_embd.bfp16) and no "
                                 "rotated ternary token_embd to restore")
            emb_mode = 2
        head_tied = head is None
        if head_tied:
            if emb is None or not L.is_ternary(emb["kind"]):
                raise ValueError("a tied LM head needs ternary token_embd rows")
            head_kind, emb_kind = emb["kind"], emb["kind"]
        else:
            head_kind = L.KIND_F16 if head["kind"] == L.KIND_F32 else head["kind"]
            emb_kind = emb["kind"] if emb is not None and L.is_ternary(emb["kind"]) else weight_kind
        cfg = make_config(mc, weight_kind, head_kind, head_tied, emb_mode, emb_kind, max_ctx, max_new, packed_ops,
                          prefill_chunk, table_free_ops)
        if rot is not None:
            block, scale, signs = rot
            cfg.hadamard_block, cfg.hadamard_scale = block, scale
            for i, w in enumerate(signs):
                cfg.hadamard_widths[i] = w
        # A rope table that is not plain RoPE (YaRN scaling) is read per position on the device.
        from .bons import image_rope_table
        t14 = image_rope_table(img)
        if t14 is not None:
            if t14.shape[0] < cfg.max_ctx:
                raise ValueError(f"the image's rope table holds {t14.shape[0]} positions, max_ctx is {cfg.max_ctx}")
            cfg.rope_table = 1
        d = cls(mc, cfg, use_graph)
        d.n_channels = img.header["n_channels"]
        d._rope_t14 = None if t14 is None else np.ascontiguousarray(t14[:cfg.max_ctx])
        try:
            d._load_image(img)
        except Exception:
            d.close()
            raise
        return d

    @classmethod
    def synthetic(cls, mc, seed=0, weight_kind=L.KIND_TERNARY5, max_ctx=None, max_new=256,
                  use_graph=True, packed_ops=PACK_AUTO, prefill_chunk=0, table_free_ops=PACK_AUTO, hadamard_block=0):
        """Fill every tensor on the device from the counter-based generator (same values as
        trixium_amd.synth.hashed_*): ternary token_embd rows (embedded by decoding the row), an
        untied ternary LM head unless the config ties them. A hybrid's DeltaNet beta|alpha Q8
        rows come from the host (seeded int8 values, fp16 scales U(0.01, 0.05)).
        hadamard_block > 0: a PrismML-rotated model (model/golden.py:250-289): every projection
        input but the DeltaNet beta/alpha rotated blockwise, scale 1/sqrt(block), random +-1 signs
        per input width (the synthetic weights stand in for weights in the rotated basis)."""
        cfg = make_config(mc, weight_kind, weight_kind, mc.tie_embeddings, 1, weight_kind, max_ctx, max_new,
                          packed_ops, prefill_chunk, table_free_ops)
        widths = []
        if hadamard_block:
            widths = sorted({mc.n_embd, mc.ffn_dim, mc.n_head * mc.head_dim}
                            | ({mc.dn_num_v_heads * mc.dn_v_head_dim} if mc.n_dn_layers else set()))
            cfg.hadamard_block, cfg.hadamard_scale = int(hadamard_block), float(1.0 / np.sqrt(hadamard_block))
            for i, w in enumerate(widths):
                cfg.hadamard_widths[i] = w
        d = cls(mc, cfg, use_graph)
        try:
            ranges = np.array([SYNTH_SCALE[0], SYNTH_SCALE[1] - SYNTH_SCALE[0],
                               SYNTH_GAIN[0], SYNTH_GAIN[1] - SYNTH_GAIN[0]], dtype=f32)
            _lib.call("trx_model_synthesize", d._h, seed & 0xFFFFFFFF,
                      ranges.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
            if mc.n_dn_layers:
                from .bons import encode_rows
                rng = np.random.default_rng(seed)
                nv = mc.dn_num_v_heads
                for l in range(mc.n_layer):
                    if mc.layer_type(l) != "deltanet":
                        continue
                    for r in (L.ROLE_SSM_BETA, L.ROLE_SSM_ALPHA):
                        q = rng.integers(-127, 128, (nv, mc.n_embd), dtype=np.int8)
                        sc = rng.uniform(0.01, 0.05, (nv, mc.n_embd // L.GROUP_Q8)).astype(np.float16)
                        d.set_tensor(r, l, encode_rows(L.KIND_Q8, mc.n_embd, sc, q))
            rng = np.random.default_rng(seed + 1)
            for i, w in enumerate(widths):
                d.set_tensor(L.ROLE_HADAMARD, i, rng.choice(np.array([-1.0, 1.0], dtype=f32), w))
        except Exception:
            d.close()
            raise
        return d

    def set_tensor(self, role, layer, arr):
        a = np.ascontiguousarray(arr)
        _lib.call("trx_model_set_tensor", self._h, role, layer, a.ctypes.data, a.nbytes)

    def _rows(self, img, e, kind):
        """Row packets of an entry in `kind` (the K-segments of a split entry joined)."""
        from .bons import decode_rows, encode_rows
        segs = img.ksegs(e)
        if len(segs) == 1 and e["kind"] == kind:
            return img.entry_rows(e)
        sc, vals = [], []
        for t in segs:
            s, v = decode_rows(t["kind"], t["cols"], img.entry_rows(t))
            sc.append(s)
            vals.append(v)
        s, v = np.concatenate(sc, axis=1), np.concatenate(vals, axis=1)
        return encode_rows(kind, v.shape[1], s, v)

    def _f32(self, img, role, layer):
        e = img.find(role, layer, L.KIND_F32)
        if e is None:
            raise ValueError(f"the image has no float32 {L.ROLE_NAMES[role]} for layer {layer}")
        return np.asarray(img.entry_tensor(e)[1], dtype=f32)

    def _load_image(self, img):
        mc, cfg = self.mc, self.cfg
        wk = cfg.weight_kind
        for l in range(mc.n_layer):
            self.set_tensor(L.ROLE_ATTN_NORM, l, self._f32(img, L.ROLE_ATTN_NORM, l))
            self.set_tensor(L.ROLE_FFN_NORM, l, self._f32(img, L.ROLE_FFN_NORM, l))
            if mc.layer_type(l) == "deltanet":
                for r in (L.ROLE_SSM_CONV, L.ROLE_SSM_A, L.ROLE_SSM_DT, L.ROLE_SSM_NORM):
                    self.set_tensor(r, l, self._f32(img, r, l))
                for r in (L.ROLE_SSM_BETA, L.ROLE_SSM_ALPHA):
                    self.set_tensor(r, l, self._rows(img, img.find(r, l), L.KIND_Q8))
                roles = _LAYER_MATRICES_DN
            else:
                for r in (L.ROLE_ATTN_Q_NORM, L.ROLE_ATTN_K_NORM):
                    self.set_tensor(r, l, self._f32(img, r, l))
                roles = _LAYER_MATRICES_ATTN
            for r in roles + _LAYER_MATRICES_FFN:
                self.set_tensor(r, l, self._rows(img, img.find(r, l), wk))
        self.set_tensor(L.ROLE_OUT_NORM, 0, self._f32(img, L.ROLE_OUT_NORM, 0))
        if getattr(self, "_rope_t14", None) is not None and mc.n_layer > mc.n_dn_layers:
            self.set_tensor(L.ROLE_ROPE_TAB, 0, self._rope_t14)
        rot = image_rotation(img)
        if rot is not None:
            for i, (w, sg) in enumerate(rot[2].items()):
                self.set_tensor(L.ROLE_HADAMARD, i, sg.astype(f32))
        if cfg.emb_mode == 0:
            _, mant = img.entry_tensor(img.find(L.ROLE_TOK_EMB16, 0))
            _, ex = img.entry_tensor(img.find(L.ROLE_TOK_EMB16_EXP, 0))
            self.set_tensor(L.ROLE_TOK_EMB16, 0, np.asarray(mant, dtype=np.int16))
            self.set_tensor(L.ROLE_TOK_EMB16_EXP, 0, np.asarray(ex).reshape(-1)[:cfg.vocab].astype(np.int32))
        if cfg.head_tied or cfg.emb_mode != 0:
            self.set_tensor(L.ROLE_TOK_EMB, 0, self._rows(img, img.find(L.ROLE_TOK_EMB, 0), cfg.emb_kind))
        if not cfg.head_tied:
            head = img.find(L.ROLE_LM_HEAD, 0)
            if cfg.head_kind == L.KIND_F16:
                w = np.asarray(img.entry_tensor(img.find(L.ROLE_LM_HEAD, 0, L.KIND_F32))[1], dtype=f32)
                self.set_tensor(L.ROLE_LM_HEAD, 0, w.astype(np.float16))
            else:
                self.set_tensor(L.ROLE_LM_HEAD, 0, self._rows(img, head, cfg.head_kind))

    def set_sampling(self, temperature=0.0, top_p=1.0, repetition=1.0, seed=0, n_channels=None):
        """Sample instead of the greedy argmax, as the firmware's `sample` does
        (firmware/infer.c:385-488): candidates are the maxima of 32 row ranges of each of
        n_channels vocabulary shards (default: the image's channel count), a repetition penalty
        over the last 64 tokens, temperature, top-p, an xorshift32 stream (seed 0 keeps it).
        temperature 0 and repetition 1 restore the greedy argmax."""
        n = int(n_channels or getattr(self, "n_channels", 1))
        _lib.call("trx_model_set_sampling", self._h, float(temperature), float(top_p), float(repetition),
                  int(seed) & 0xFFFFFFFF, n)

    # State and decoding ------------------------------------------------------------------------
    def reset(self):
        _lib.call("trx_model_reset", self._h)

    def checkpoint(self):
        """Save the decode state after the work enqueued so far (position, fed and generated
        tokens, argmax slot, sampler stream, DeltaNet conv windows and recurrent state), as the
        firmware's hybrid_ckpt_save does before a forward it may run again
        (firmware/hybrid.c:2904-2930, infer.c:1926-1960 forward_checked)."""
        _lib.call("trx_model_checkpoint", self._h, CKPT_SAVE)

    def set_kv_ring(self, enable=-1, pin=4):
        """The KV ring past max_ctx (firmware/hybrid.c:156-181, the console's `kvring` and
        hybrid_set_pin), from the next reset on: the first `pin` positions stay (4 to max_ctx/4)
        and the rest of the window is a ring of the most recent positions, so forwards go on past
        max_ctx. enable: 1 on, 0 off, -1 the default (on for a model with DeltaNet layers)."""
        _lib.call("trx_model_set_kv_ring", self._h, int(enable), int(pin))

    @property
    def kv_pin(self):
        """Positions the KV ring keeps past the window since the last reset (0: no ring)."""
        return self.info(INFO_KV_PIN)

    def restore(self):
        """Put the last checkpoint's state back: the next forwards give the results they gave
        after checkpoint() (KV rows past the position are rewritten before they are read)."""
        _lib.call("trx_model_checkpoint", self._h, CKPT_RESTORE)

    def feed(self, tokens, head_from=-1):
        """Queue tokens for the next len(tokens) positions; the forwards run on step()."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        if t.size == 0:
            raise ValueError("no tokens to feed")
        _lib.call("trx_model_set_prompt", self._h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                  int(t.size), int(head_from))
        return t.size

    def step(self, n_steps, use_graph=None):
        """Enqueue n forwards (one position each); returns without waiting."""
        g = self.use_graph if use_graph is None else use_graph
        _lib.call("trx_model_step", self._h, int(n_steps), int(bool(g)))

    def prefill(self, n, chunk=0):
        """Enqueue the batched prefill of the next n fed positions, `chunk` positions per weight
        pass (0: the config's prefill_chunk, else 1024); they must precede the first position
        that computes logits. The state afterwards is that of n one-position forwards."""
        c = int(chunk or self.cfg.prefill_chunk or 1024)
        _lib.call("trx_model_prefill", self._h, int(n), c)

    def _run_fed(self, n, extra, use_graph):
        # n fed tokens, then `extra` more positions: all but the last fed one through the batched
        # prefill when the config asks for it.
        pre = n - 1 if self.cfg.prefill_chunk > 0 else 0
        if pre:
            self.prefill(pre)
        self.step(n - pre + extra, use_graph)

    def forward(self, tokens, use_graph=None):
        """Feed `tokens` after the current position; logits (vocab,) of the last one
        (FloatModel.forward, golden.py:436-460)."""
        n = self.feed(tokens)
        self._run_fed(n, 0, use_graph)
        return self.logits()

    def generate(self, tokens, n, use_graph=None):
        """Greedy continuation of `tokens` after the current position; the n generated ids
        (FloatModel.generate, golden.py:462-470)."""
        if n <= 0:
            return []
        if n > self.cfg.max_new:
            raise ValueError(f"{n} tokens requested, the output buffer holds {self.cfg.max_new}")
        n_fed = self.feed(tokens)
        self._run_fed(n_fed, n - 1, use_graph)
        self.finalize()
        return [int(v) for v in self.outputs()[:n]]

    def generate_fresh(self, prompt, n, use_graph=None):
        """reset + generate through the single C entry point (firmware infer_generate)."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        out = np.empty(n, dtype=np.int32)
        g = self.use_graph if use_graph is None else use_graph
        _lib.call("trx_model_generate", self._h, p.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                  int(p.size), int(n), out.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), int(bool(g)))
        return [int(v) for v in out]

    def outputs(self):
        """The generated-token buffer (int32 [max_new]) after finalize()."""
        return self._read(READ_OUT, np.empty(self.cfg.max_new, dtype=np.int32))

    def finalize(self):
        """Resolve the argmax of the last forward into the output buffer."""
        _lib.call("trx_model_finalize", self._h)

    def synchronize(self):
        _lib.call("trx_model_sync", self._h)

    def _read(self, what, arr):
        _lib.call("trx_model_read", self._h, what, arr.ctypes.data, arr.nbytes)
        return arr

    def logits(self, Hs=None):
        """Without arguments: the logits (vocab,) of the last forward that ran the LM head. With
        hidden states Hs [T, n_embd]: the LM head applied to them on the GPU, [T, vocab]
        (HybridRef.logits, model/fastref.py:260-261)."""
        if Hs is None:
            return self._read(READ_LOGITS, np.empty(self.vocab, dtype=f32))
        h = np.ascontiguousarray(np.asarray(Hs, dtype=f32).reshape(-1, self.n_embd))
        out = np.empty((h.shape[0], self.vocab), dtype=f32)
        _lib.call("trx_model_project_head", self._h, h.ctypes.data, int(h.shape[0]), out.ctypes.data)
        return out

    def hidden(self, tokens=None):
        """Without arguments: the final normed hidden state (n_embd,) of the last forward. With
        tokens: reset, run them teacher-forced from position 0 and return every position's final
        normed hidden state [T, n_embd] (HybridRef.hidden, model/fastref.py:244-258)."""
        if tokens is None:
            return self._read(READ_HIDDEN, np.empty(self.n_embd, dtype=f32))
        return self.score(tokens)[1]

    def residual(self):
        """The residual stream (n_embd,) after the last layer of the last forward (un-normed)."""
        return self._read(READ_RESIDUAL, np.empty(self.n_embd, dtype=f32))

    def score(self, tokens, chunk=256):
        """(nll [T-1] of tokens[1:] given their prefix, final normed hidden states [T, n_embd]),
        teacher-forced from position 0 after a reset (HybridRef.score, model/fastref.py:263-273).
        The log-sum-exp over the vocabulary runs on the GPU in float32; `chunk` is accepted for
        the reference's signature (the GPU scores one position at a time)."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        if t.size == 0:
            raise ValueError("no tokens to score")
        nll = np.empty(max(t.size - 1, 1), dtype=f32)
        hid = np.empty((t.size, self.n_embd), dtype=f32)
        _lib.call("trx_model_score", self._h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), int(t.size),
                  nll.ctypes.data, hid.ctypes.data)
        return nll[:t.size - 1].astype(np.float64), hid

    def taps(self):
        """Intermediate vectors of the last forward: the last attention layer's q|k|v projection
        and attention output, and the last layer's SwiGLU activation (float32)."""
        c = self.cfg
        nq = c.n_head * c.head_dim * (2 if c.attn_gated else 1) + 2 * c.n_kv_head * c.head_dim
        return {"qkv": self._read(READ_QKV, np.empty(nq, dtype=f32)),
                "attn": self._read(READ_ATTN, np.empty(c.n_head * c.head_dim, dtype=f32)),
                "act": self._read(READ_ACT, np.empty(c.ffn_dim, dtype=f32))}

    def position(self):
        """Position of the last forward (-1 after reset)."""
        return int(self._read(READ_POSITION, np.empty(1, dtype=np.int32))[0])

    def info(self, what):
        v = ctypes.c_int64()
        _lib.call("trx_model_info", self._h, what, ctypes.byref(v))
        return v.value

    @property
    def attention_splits(self):
        """(position splits per kv head, positions per pass of a split block) of the decode
        attention: a split of c positions takes ceil(c / positions per pass) passes."""
        return self.info(INFO_ATTN_SPLITS), self.info(INFO_ATTN_PASS)

    @property
    def stream(self):
        return self.info(INFO_STREAM)

    @property
    def packed_ops(self):
        """TRX_PACK_* bits of the projections that run on the packed GEMV."""
        return self.info(INFO_PACKED_OPS)

    @property
    def table_free_ops(self):
        """TRX_PACK_* bits of the packed projections on the table-free lookups."""
        return self.info(INFO_TABLE_FREE_OPS)

    def packed_ptr(self, op, layer=0):
        """(packed copy, shared workspace) device addresses of one packed projection."""
        p, w = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("trx_model_packed_ptr", self._h, op, layer, ctypes.byref(p), ctypes.byref(w))
        return p.value, w.value

    def tensor_ptr(self, role, layer=0):
        p, n = ctypes.c_void_p(), ctypes.c_int64()
        _lib.call("trx_model_tensor_ptr", self._h, role, layer, ctypes.byref(p), ctypes.byref(n))
        return p.value, n.value

    def read_tensor(self, role, layer=0):
        """Raw bytes of a resident tensor (uint8)."""
        p, n = self.tensor_ptr(role, layer)
        out = np.empty(n, dtype=np.uint8)
        self.synchronize()
        _lib.call("trx_memcpy_d2h", out.ctypes.data, p, n, None)
        _lib.call("trx_stream_sync", None)
        return out

    def close(self):
        if getattr(self, "_h", None):
            _lib.lib().trx_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
