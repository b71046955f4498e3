"""Float reference of the ternary decoder (test infrastructure only, see oracle/__init__.py).

The arithmetic is model/fastref.py's (HybridRef: fp32 activations, weights dequantised as
(code - 1) * scale and held in fp16, which is exact for ternary; embedding rows from the int16
BFP table; plain RoPE with float32 angles; NEOX pairs on the first rope_dims of a head). An
image whose rope table is not plain RoPE (YaRN scaling, which exists only in that table) rotates
with the table's Q14 cos/sin per position instead, as the firmware and model/mirror.py:478-483
do; fastref ignores the table. The
state semantics are model/golden.py:FloatModel's (K/V caches appended post-norm/post-RoPE (K)
and raw (V), a (K-1)-deep conv window and a per-value-head fp32 recurrent matrix for every
DeltaNet layer, `pos` advanced per forward), so the reference steps one token at a time like
the GPU loop does. `kv_fp16=True` rounds cached K/V to fp16 as the GPU cache stores them.
"""

import numpy as np

from trixium_amd import layout as L

f32 = np.float32


class FloatRef:
    # KV ring past the window (set_kv_ring): off unless asked for.
    ring_cap, ring_pin_next, ring_window, kv_pin = None, 4, False, 0

    def __init__(self, img, kv_fp16=False):
        self.img = img
        h = self.h = img.header
        self.n_layer, self.n_embd = h["n_layer"], h["n_embd"]
        self.n_head, self.n_kv, self.hd = h["n_head"], h["n_kv_head"], h["head_dim"]
        self.nk, self.hk = h["dn_num_k_heads"], h["dn_k_head_dim"]
        self.nv, self.hv = h["dn_num_v_heads"], h["dn_v_head_dim"]
        self.K = h["dn_conv_kernel"]
        self.rope_n = h["rope_dims"] or self.hd
        self.eps = f32(h["rms_eps"])
        self.gated = bool(h["attn_gated"])
        self.vocab = h["vocab"]
        self.dn = [t == "deltanet" for t in h["layer_types"]]
        # PrismML's rotated basis: every ternary projection's input goes through the image's
        # rotation tensors first (fastref.py:127-140), the DeltaNet beta/alpha excepted.
        self.hb, self.hwidths = h["hadamard_block"], list(h["hadamard_widths"])
        self.kv_fp16 = kv_fp16
        self.wcache = {}
        # fastref.py:62-63: theta**(-2i/n) evaluated in float32.
        self.rope_freq = np.array([f32(f32(h["rope_theta"]) ** f32(-2.0 * i / self.rope_n))
                                   for i in range(self.rope_n // 2)], dtype=f32)
        from trixium_amd.bons import image_rope_table
        self.rope_tab = image_rope_table(img)
        self.norm_attn = [self._f32(L.ROLE_ATTN_NORM, l) for l in range(self.n_layer)]
        self.norm_ffn = [self._f32(L.ROLE_FFN_NORM, l) for l in range(self.n_layer)]
        self.norm_q, self.norm_k, self.norm_ssm, self.ssm_a, self.ssm_dt, self.conv_w = {}, {}, {}, {}, {}, {}
        for l in range(self.n_layer):
            if self.dn[l]:
                self.norm_ssm[l] = self._f32(L.ROLE_SSM_NORM, l)
                self.ssm_a[l] = self._f32(L.ROLE_SSM_A, l)
                self.ssm_dt[l] = self._f32(L.ROLE_SSM_DT, l)
                self.conv_w[l] = self._f32(L.ROLE_SSM_CONV, l).reshape(-1, self.K)
            else:
                self.norm_q[l] = self._f32(L.ROLE_ATTN_Q_NORM, l)
                self.norm_k[l] = self._f32(L.ROLE_ATTN_K_NORM, l)
        self.out_norm = self._f32(L.ROLE_OUT_NORM, 0)
        self.head_role = L.ROLE_LM_HEAD if img.find(L.ROLE_LM_HEAD, 0) else L.ROLE_TOK_EMB
        e16 = img.find(L.ROLE_TOK_EMB16, 0)
        if e16 is not None:
            _, self.emb_mant = img.entry_tensor(e16)
            _, ex = img.entry_tensor(img.find(L.ROLE_TOK_EMB16_EXP, 0))
            self.emb_exp = np.asarray(ex).reshape(-1)
            self.emb_restore = None
        else:
            # No int16 table: each row of the rotated token_embd is restored to the plain basis
            # in integers (fastref.py:173-177, bons.py:262-295); the signs are row 0 of each
            # rotation block of the n_embd width (R[0] = +1).
            assert self.hb, "an image without the int16 table must be rotated"
            wi = self.hwidths.index(self.n_embd)
            signs = np.concatenate([
                np.asarray(img.entry_tensor(img.find(L.ROLE_HADAMARD, L.hadamard_layer(wi, b)))[1])[0]
                .astype(np.int64) - 1 for b in range(self.n_embd // self.hb)])
            sc, codes = img.entry_tensor(img.find(L.ROLE_TOK_EMB, 0))
            self.emb_restore = (np.asarray(sc), np.asarray(codes), signs)
        self.reset()

    # Tensors (fastref.py:86-125) -----------------------------------------------------------
    def _f32(self, role, l):
        e = self.img.find(role, l, L.KIND_F32)
        assert e is not None, (role, l)
        return np.asarray(self.img.entry_tensor(e)[1], dtype=f32).reshape(-1)

    def weight(self, role, l):
        key = (role, l)
        if key not in self.wcache:
            e = self.img.find(role, l)
            ws = []
            for t in self.img.ksegs(e):
                scales, codes = self.img.entry_tensor(t)
                if t["kind"] == L.KIND_F32:
                    ws.append(np.asarray(codes, dtype=f32).reshape(t["rows"], t["cols"]))
                    continue
                g = 128 if L.is_ternary(t["kind"]) else 32
                off = f32(1.0) if L.is_ternary(t["kind"]) else f32(0.0)
                w = (codes.astype(f32).reshape(t["rows"], -1, g) - off) * scales.astype(f32)[:, :, None]
                ws.append(w.reshape(t["rows"], t["cols"]))
            self.wcache[key] = np.concatenate(ws, axis=1).astype(np.float16)
        return self.wcache[key]

    def rotate(self, x, width):
        """x' = the rotation blocks (ternary block x block tensors) applied blockwise."""
        out = np.empty(width, f32)
        wi = self.hwidths.index(width)
        for b in range(width // self.hb):
            W = self.weight(L.ROLE_HADAMARD, L.hadamard_layer(wi, b))
            out[b * self.hb:(b + 1) * self.hb] = W.astype(f32) @ x[b * self.hb:(b + 1) * self.hb]
        return out

    def proj(self, role, l, x):
        """W x in fp32 from the fp16 weight cache, 8192 rows at a time (fastref.py:119-125)."""
        W = self.weight(role, l)
        x = np.asarray(x, dtype=f32)
        if self.hb and role not in (L.ROLE_SSM_BETA, L.ROLE_SSM_ALPHA):
            x = self.rotate(x, W.shape[1])
        out = np.empty(W.shape[0], f32)
        for r0 in range(0, W.shape[0], 8192):
            out[r0:r0 + 8192] = W[r0:r0 + 8192].astype(f32) @ x
        return out

    # Elementwise ops (fastref.py:143-156) ----------------------------------------------------
    def rmsnorm(self, x, w):
        r = f32(1.0) / np.sqrt((x * x).mean(axis=-1, keepdims=True, dtype=f32) + self.eps)
        return (x * r * w).astype(f32)

    def l2norm(self, x):
        n = np.maximum(np.sqrt((x * x).sum(axis=-1, keepdims=True, dtype=f32)), self.eps)
        return (x / n).astype(f32)

    @staticmethod
    def sigmoid(x):
        with np.errstate(over="ignore"):       # exp(-x) = inf for x << 0 gives the exact 0
            return (f32(1.0) / (f32(1.0) + np.exp(-x))).astype(f32)

    @staticmethod
    def silu(x):
        return (x / (f32(1.0) + np.exp(-x))).astype(f32)

    @staticmethod
    def softplus(x):
        return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20)))).astype(f32)

    # State (golden.py:304-320) ---------------------------------------------------------------
    def set_kv_ring(self, ctx_cap, pin=4, window=False):
        """From the next reset: keep ctx_cap KV slots per layer, past them the first `pin`
        positions (4 to ctx_cap // 4, firmware/hybrid.c:1148-1149) and a ring of the most recent
        ones in the rest (kv_slot, hybrid.c:176-181), every slot attended (hybrid.c:2483); the ring
        only where ctx_cap > 2 pin (kv_ring_on, hybrid.c:170-173). ctx_cap None: no ring.
        window=True keeps every row instead and attends the positions the ring keeps, [0, pin) and
        the last ctx_cap - pin (the ring's specification, for checking it)."""
        self.ring_cap, self.ring_pin_next, self.ring_window = ctx_cap, pin, window

    def reset(self):
        self.kv_pin = 0
        if self.ring_cap is not None:
            pin = max(4, min(self.ring_pin_next, self.ring_cap // 4))
            self.kv_pin = pin if self.ring_cap > 2 * pin else 0
        self.pos = 0
        self.k_cache = {l: [] for l in range(self.n_layer) if not self.dn[l]}
        self.v_cache = {l: [] for l in range(self.n_layer) if not self.dn[l]}
        C = 2 * self.nk * self.hk + self.nv * self.hv
        self.conv_state = {l: np.zeros((self.K - 1, C), f32) for l in range(self.n_layer) if self.dn[l]}
        self.dn_state = {l: np.zeros((self.nv, self.hv, self.hk), f32) for l in range(self.n_layer) if self.dn[l]}

    def embed(self, tok):
        if getattr(self, "emb_restore", None) is not None:
            from .bitexact import restored_row_exact
            sc, codes, signs = self.emb_restore
            m, e = restored_row_exact(sc[tok], codes[tok], signs, self.hb)
            return (m.astype(f32) * f32(np.exp2(e))).astype(f32)
        return (self.emb_mant[tok].astype(f32) * f32(np.exp2(int(self.emb_exp[tok])))).astype(f32)

    def attention(self, l, hn, pos):
        hd, nh, nkv = self.hd, self.n_head, self.n_kv
        qf = self.proj(L.ROLE_ATTN_Q, l, hn)
        k = self.proj(L.ROLE_ATTN_K, l, hn).reshape(nkv, hd)
        v = self.proj(L.ROLE_ATTN_V, l, hn).reshape(nkv, hd)
        if self.gated:
            qf = qf.reshape(nh, 2 * hd)
            q, gate = qf[:, :hd], qf[:, hd:]
        else:
            q, gate = qf.reshape(nh, hd), None
        q = self.rmsnorm(q, self.norm_q[l])
        k = self.rmsnorm(k, self.norm_k[l])
        half = self.rope_n // 2
        if getattr(self, "rope_tab", None) is not None:
            row = self.rope_tab[pos].astype(f32) * f32(2.0**-14)
            cos, sin = row[:half], row[half:]
        else:
            ang = (f32(pos) * self.rope_freq).astype(f32)
            cos, sin = np.cos(ang), np.sin(ang)

        def rope(x):
            x = x.copy()
            x0, x1 = x[:, :half].copy(), x[:, half:self.rope_n].copy()
            x[:, :half] = x0 * cos - x1 * sin
            x[:, half:self.rope_n] = x0 * sin + x1 * cos
            return x

        q, k = rope(q), rope(k)
        q = (q * f32(1.0 / np.sqrt(hd))).astype(f32)
        if self.kv_fp16:
            k, v = k.astype(np.float16).astype(f32), v.astype(np.float16).astype(f32)
        cap, pin = self.ring_cap, self.kv_pin
        if pin and pos >= cap and not self.ring_window:
            slot = pin + (pos - pin) % (cap - pin)  # firmware/hybrid.c:176-181 kv_slot
            self.k_cache[l][slot] = k
            self.v_cache[l][slot] = v
        else:
            self.k_cache[l].append(k)
            self.v_cache[l].append(v)
        Kc = np.stack(self.k_cache[l])             # [T, nkv, hd]
        Vc = np.stack(self.v_cache[l])
        if pin and pos >= cap and self.ring_window:
            keep = np.r_[0:pin, pos - (cap - pin) + 1:pos + 1]
            Kc, Vc = Kc[keep], Vc[keep]
        rep = nh // nkv
        out = np.empty((nh, hd), f32)
        for h in range(nh):
            s = (Kc[:, h // rep] @ q[h]).astype(f32)
            s = s - s.max()
            p = np.exp(s)
            p = (p / p.sum()).astype(f32)
            out[h] = (p @ Vc[:, h // rep]).astype(f32)
        if gate is not None:
            out = (out * self.sigmoid(gate)).astype(f32)
        return self.proj(L.ROLE_ATTN_OUT, l, out.reshape(-1))

    def deltanet(self, l, hn):
        """One position of the gated delta rule (fastref.py:182-214, golden.py:400-434)."""
        nq = self.nk * self.hk
        qkv = self.proj(L.ROLE_ATTN_QKV, l, hn)
        z = self.proj(L.ROLE_ATTN_ZGATE, l, hn)
        beta = self.sigmoid(self.proj(L.ROLE_SSM_BETA, l, hn))
        alpha = self.proj(L.ROLE_SSM_ALPHA, l, hn)
        decay = np.exp((self.softplus(alpha + self.ssm_dt[l]) * self.ssm_a[l]).astype(f32))
        w = self.conv_w[l]
        win = np.concatenate([self.conv_state[l], qkv[None, :]], axis=0)      # [K, C]
        conv = sum(win[i] * w[:, i] for i in range(self.K)).astype(f32)
        self.conv_state[l] = win[1:].copy()
        conv = self.silu(conv)
        q = self.l2norm(conv[:nq].reshape(self.nk, self.hk))
        k = self.l2norm(conv[nq:2 * nq].reshape(self.nk, self.hk))
        v = conv[2 * nq:].reshape(self.nv, self.hv)
        kh = np.arange(self.nv) % self.nk
        M = self.dn_state[l]
        qt, kt = q[kh], k[kh]
        M *= decay[:, None, None]
        delta = (v - np.einsum("hjk,hk->hj", M, kt)) * beta[:, None]
        M += delta[:, :, None] * kt[:, None, :]
        o = (np.einsum("hjk,hk->hj", M, qt) * f32(1.0 / np.sqrt(self.hk))).astype(f32)
        nrm = self.rmsnorm(o, self.norm_ssm[l])
        gz = nrm * self.silu(z.reshape(self.nv, self.hv))
        rep = self.nv // self.nk
        gpos = kh * rep + np.arange(self.nv) // self.nk
        og = np.empty_like(gz)
        og[gpos] = gz
        return self.proj(L.ROLE_SSM_OUT, l, og.reshape(-1).astype(f32))

    def step(self, tok, want_logits=True):
        """One decode position: residual stream through every layer, then (optionally) the
        logits over the vocabulary (fastref.py:244-261 per position)."""
        x = self.embed(tok)
        for l in range(self.n_layer):
            hn = self.rmsnorm(x, self.norm_attn[l])
            y = self.deltanet(l, hn) if self.dn[l] else self.attention(l, hn, self.pos)
            x = (x + y).astype(f32)
            hn = self.rmsnorm(x, self.norm_ffn[l])
            g = self.proj(L.ROLE_FFN_GATE, l, hn)
            u = self.proj(L.ROLE_FFN_UP, l, hn)
            x = (x + self.proj(L.ROLE_FFN_DOWN, l, (self.silu(g) * u).astype(f32))).astype(f32)
        self.pos += 1
        self.last_hidden = x
        if not want_logits:
            return None
        hn = self.rmsnorm(x, self.out_norm)
        return self.proj(self.head_role, 0, hn)[:self.vocab]

    def score(self, tokens):
        """(nll [T-1], final normed hidden states [T, n_embd]) of a sequence teacher-forced from
        position 0 after a reset (fastref.py:244-273: hidden = rmsnorm(residual, out_norm); the
        log-sum-exp of every position's logits in float64)."""
        self.reset()
        nll, hid = [], []
        for i, t in enumerate(tokens):
            lg = self.step(int(t), want_logits=i + 1 < len(tokens))
            hid.append(self.rmsnorm(self.last_hidden, self.out_norm))
            if lg is not None:
                l64 = lg.astype(np.float64)
                m = l64.max()
                nll.append(m + np.log(np.exp(l64 - m).sum()) - l64[int(tokens[i + 1])])
        return np.array(nll, np.float64), np.stack(hid)

    def forward(self, tokens):
        """FloatModel.forward contract (golden.py:436-460): logits of the last position."""
        logits = None
        for i, t in enumerate(tokens):
            logits = self.step(int(t), want_logits=(i == len(tokens) - 1))
        return logits

    def generate(self, prompt, n_new):
        """Greedy decode with the firmware loop contract (mirror.py:1036-1044): prefill one token
        per forward, logits only at the last prompt position, no forward after the last output."""
        out = []
        logits = self.forward(prompt)
        for i in range(n_new):
            nxt = int(np.argmax(logits))
            out.append(nxt)
            if i + 1 < n_new:
                logits = self.step(nxt)
        return out

    # Whole-sequence forward (fastref.py:244-258: every projection of a layer over all positions
    # at once, causal attention over the sequence) --------------------------------------------
    def proj_many(self, role, l, X):
        """Rows X [T, cols] -> [T, rows]: fastref's X @ W.T (fastref.py:119-125)."""
        W = self.weight(role, l)
        X = np.asarray(X, dtype=f32)
        if self.hb and role not in (L.ROLE_SSM_BETA, L.ROLE_SSM_ALPHA):
            X = np.stack([self.rotate(x, W.shape[1]) for x in X])
        return (X @ W.astype(f32).T).astype(f32)

    def _rope_rows(self, positions):
        half = self.rope_n // 2
        if getattr(self, "rope_tab", None) is not None:
            rows = self.rope_tab[positions].astype(f32) * f32(2.0**-14)
            return rows[:, :half], rows[:, half:]
        ang = (positions.astype(f32)[:, None] * self.rope_freq[None, :]).astype(f32)
        return np.cos(ang), np.sin(ang)

    def attention_many(self, l, Hn, pos0):
        """Positions pos0 .. pos0 + T - 1 of one attention layer, each attending to the cached
        positions and to the sequence's positions up to itself (fastref.py:216-241)."""
        T = Hn.shape[0]
        hd, nh, nkv = self.hd, self.n_head, self.n_kv
        qf = self.proj_many(L.ROLE_ATTN_Q, l, Hn)
        k = self.proj_many(L.ROLE_ATTN_K, l, Hn).reshape(T, nkv, hd)
        v = self.proj_many(L.ROLE_ATTN_V, l, Hn).reshape(T, nkv, hd)
        if self.gated:
            qf = qf.reshape(T, nh, 2 * hd)
            q, gate = qf[:, :, :hd], qf[:, :, hd:]
        else:
            q, gate = qf.reshape(T, nh, hd), None
        q = self.rmsnorm(q, self.norm_q[l])
        k = self.rmsnorm(k, self.norm_k[l])
        half = self.rope_n // 2
        cos, sin = self._rope_rows(pos0 + np.arange(T))
        cos, sin = cos[:, None, :], sin[:, None, :]

        def rope(x):
            x = x.copy()
            x0, x1 = x[:, :, :half].copy(), x[:, :, half:self.rope_n].copy()
            x[:, :, :half] = x0 * cos - x1 * sin
            x[:, :, half:self.rope_n] = x0 * sin + x1 * cos
            return x

        q, k = rope(q), rope(k)
        q = (q * f32(1.0 / np.sqrt(hd))).astype(f32)
        if self.kv_fp16:
            k, v = k.astype(np.float16).astype(f32), v.astype(np.float16).astype(f32)
        P = len(self.k_cache[l])
        self.k_cache[l].extend(list(k))
        self.v_cache[l].extend(list(v))
        Kc = np.stack(self.k_cache[l])             # [P + T, nkv, hd]
        Vc = np.stack(self.v_cache[l])
        rep = nh // nkv
        # Query i (position pos0 + i) sees cache rows 0 .. P + i.
        future = np.arange(P + T)[None, :] > (P + np.arange(T))[:, None]
        out = np.empty((T, nh, hd), f32)
        for h in range(nh):
            s = (q[:, h] @ Kc[:, h // rep].T).astype(f32)
            s[future] = -np.inf
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p = (p / p.sum(axis=1, keepdims=True)).astype(f32)
            out[:, h] = (p @ Vc[:, h // rep]).astype(f32)
        if gate is not None:
            out = (out * self.sigmoid(gate)).astype(f32)
        return self.proj_many(L.ROLE_ATTN_OUT, l, out.reshape(T, -1))

    def deltanet_many(self, l, Hn):
        """The gated delta rule over T positions (fastref.py:182-214): projections and the conv
        over the whole sequence, the recurrence position by position."""
        T = Hn.shape[0]
        nq = self.nk * self.hk
        qkv = self.proj_many(L.ROLE_ATTN_QKV, l, Hn)
        z = self.proj_many(L.ROLE_ATTN_ZGATE, l, Hn)
        beta = self.sigmoid(self.proj_many(L.ROLE_SSM_BETA, l, Hn))
        alpha = self.proj_many(L.ROLE_SSM_ALPHA, l, Hn)
        decay = np.exp((self.softplus(alpha + self.ssm_dt[l]) * self.ssm_a[l]).astype(f32))
        w = self.conv_w[l]
        win = np.concatenate([self.conv_state[l], qkv], axis=0)                # [K - 1 + T, C]
        conv = sum(win[i:i + T] * w[:, i] for i in range(self.K)).astype(f32)
        self.conv_state[l] = win[T:].copy()
        conv = self.silu(conv)
        kh = np.arange(self.nv) % self.nk
        rep = self.nv // self.nk
        gpos = kh * rep + np.arange(self.nv) // self.nk
        M = self.dn_state[l]
        og = np.empty((T, self.nv * self.hv), f32)
        for t in range(T):
            q = self.l2norm(conv[t, :nq].reshape(self.nk, self.hk))
            k = self.l2norm(conv[t, nq:2 * nq].reshape(self.nk, self.hk))
            v = conv[t, 2 * nq:].reshape(self.nv, self.hv)
            qt, kt = q[kh], k[kh]
            M *= decay[t][:, None, None]
            delta = (v - np.einsum("hjk,hk->hj", M, kt)) * beta[t][:, None]
            M += delta[:, :, None] * kt[:, None, :]
            o = (np.einsum("hjk,hk->hj", M, qt) * f32(1.0 / np.sqrt(self.hk))).astype(f32)
            gz = self.rmsnorm(o, self.norm_ssm[l]) * self.silu(z[t].reshape(self.nv, self.hv))
            row = np.empty_like(gz)
            row[gpos] = gz
            og[t] = row.reshape(-1)
        return self.proj_many(L.ROLE_SSM_OUT, l, og)

    def prefill(self, tokens, want_logits=False):
        """Run `tokens` at the next len(tokens) positions as one teacher-forced sequence
        (fastref.py:244-258's whole-sequence form; the caches, conv windows and recurrent states
        end as after that many step() calls). Returns the last position's logits when asked."""
        pos0 = self.pos
        assert not (self.kv_pin and pos0 + len(tokens) > self.ring_cap), "past the KV window: step()"
        X = np.stack([self.embed(int(t)) for t in tokens]).astype(f32)
        for l in range(self.n_layer):
            hn = self.rmsnorm(X, self.norm_attn[l])
            y = self.deltanet_many(l, hn) if self.dn[l] else self.attention_many(l, hn, pos0)
            X = (X + y).astype(f32)
            hn = self.rmsnorm(X, self.norm_ffn[l])
            g = self.proj_many(L.ROLE_FFN_GATE, l, hn)
            u = self.proj_many(L.ROLE_FFN_UP, l, hn)
            X = (X + self.proj_many(L.ROLE_FFN_DOWN, l, (self.silu(g) * u).astype(f32))).astype(f32)
        self.pos += len(tokens)
        self.last_hidden = X[-1]
        if not want_logits:
            return None
        hn = self.rmsnorm(X[-1], self.out_norm)
        return self.proj(self.head_role, 0, hn)[:self.vocab]


class ShapeSample(FloatRef):
    """FloatRef's decode step on random weights of a model shape, built without an image (the CPU
    baseline of a large model is timed on a sample of its layers).

    Weights are ternary-valued fp16 matrices ((code - 1) * scale, scales U(0.01, 0.05)), the
    embedding table random int16 mantissas, the KV caches filled with `ctx` random positions, so
    the next step() runs at position `ctx` with the per-token work of the full shape restricted to
    `n_layer` layers. `kinds` gives the sample layers' kinds ("attn" or "deltanet"; default all
    attention): a DeltaNet layer gets the shape's conv, gates and a random recurrent state."""

    def __init__(self, mc, n_layer, ctx, seed=0, kinds=None):
        rng = np.random.default_rng(seed)
        kinds = list(kinds or ["attn"] * n_layer)
        assert len(kinds) == n_layer
        self.n_layer, self.n_embd = n_layer, mc.n_embd
        self.n_head, self.n_kv, self.hd = mc.n_head, mc.n_kv_head, mc.head_dim
        self.rope_n = mc.rope_dims or mc.head_dim
        self.eps = f32(mc.rms_eps)
        self.gated = bool(mc.attn_gated)
        self.hb, self.hwidths = 0, []          # plain basis
        self.vocab = mc.vocab
        self.dn = [k == "deltanet" for k in kinds]
        self.nk, self.hk = mc.dn_num_k_heads, mc.dn_k_head_dim
        self.nv, self.hv = mc.dn_num_v_heads, mc.dn_v_head_dim
        self.K = mc.dn_conv_kernel if any(self.dn) else 1
        self.kv_fp16 = True
        self.rope_freq = np.array([f32(f32(mc.rope_theta) ** f32(-2.0 * i / self.rope_n))
                                   for i in range(self.rope_n // 2)], dtype=f32)

        def tern(rows, cols):
            # A block of up to 1024 random rows repeated down the matrix: the step's cost does
            # not depend on the values, and building a 151936-row head stays fast.
            b = min(rows, 1024)
            w = rng.integers(-1, 2, size=(b, cols), dtype=np.int8).astype(np.float16)
            s = rng.uniform(0.01, 0.05, size=(b, cols // 128, 1)).astype(np.float16)
            blk = (w.reshape(b, -1, 128) * s).reshape(b, cols)
            return np.tile(blk, (-(-rows // b), 1))[:rows]

        E, q, kv, F = mc.n_embd, mc.n_head * mc.head_dim, mc.n_kv_head * mc.head_dim, mc.ffn_dim
        nq, nvh = self.nk * self.hk, self.nv * self.hv
        self.wcache = {}
        for l in range(n_layer):
            if self.dn[l]:
                mats = ((L.ROLE_ATTN_QKV, 2 * nq + nvh, E), (L.ROLE_ATTN_ZGATE, nvh, E),
                        (L.ROLE_SSM_BETA, self.nv, E), (L.ROLE_SSM_ALPHA, self.nv, E), (L.ROLE_SSM_OUT, E, nvh))
            else:
                mats = ((L.ROLE_ATTN_Q, q * (2 if self.gated else 1), E), (L.ROLE_ATTN_K, kv, E),
                        (L.ROLE_ATTN_V, kv, E), (L.ROLE_ATTN_OUT, E, q))
            for role, r, c in mats + ((L.ROLE_FFN_GATE, F, E), (L.ROLE_FFN_UP, F, E), (L.ROLE_FFN_DOWN, E, F)):
                self.wcache[(role, l)] = tern(r, c)
        self.head_role = L.ROLE_LM_HEAD
        self.wcache[(L.ROLE_LM_HEAD, 0)] = tern(mc.vocab, E)
        gain = lambda n: rng.uniform(0.8, 1.2, n).astype(f32)
        self.norm_attn = [gain(E) for _ in range(n_layer)]
        self.norm_ffn = [gain(E) for _ in range(n_layer)]
        self.norm_q = {l: gain(mc.head_dim) for l in range(n_layer) if not self.dn[l]}
        self.norm_k = {l: gain(mc.head_dim) for l in range(n_layer) if not self.dn[l]}
        dls = [l for l in range(n_layer) if self.dn[l]]
        self.norm_ssm = {l: gain(self.hv) for l in dls}
        self.ssm_a = {l: -np.exp(rng.uniform(-1.5, 0.5, self.nv)).astype(f32) for l in dls}
        self.ssm_dt = {l: rng.uniform(-2.0, 0.5, self.nv).astype(f32) for l in dls}
        self.conv_w = {l: rng.uniform(-0.5, 0.5, (2 * nq + nvh, self.K)).astype(f32) for l in dls}
        self.out_norm = gain(E)
        self.emb_mant = np.tile(rng.integers(-32767, 32768, size=(256, E), dtype=np.int16),
                                (-(-mc.vocab // 256), 1))[:mc.vocab]
        self.emb_exp = np.full(mc.vocab, -20, np.int32)
        self.reset()
        for l in dls:
            self.dn_state[l] = (0.1 * rng.standard_normal((self.nv, self.hv, self.hk))).astype(f32)
        for l in range(n_layer):
            if self.dn[l]:
                continue
            kc = rng.standard_normal((ctx, self.n_kv, self.hd)).astype(np.float16).astype(f32)
            vc = rng.standard_normal((ctx, self.n_kv, self.hd)).astype(np.float16).astype(f32)
            self.k_cache[l] = list(kc)
            self.v_cache[l] = list(vc)
        self.pos = ctx


class TensorRef(FloatRef):
    """FloatRef's step over weights given as arrays instead of an image: the headline shapes (and
    the hybrid's layer pattern), whose weights the device generator fills in HBM and a test reads
    back.

    weights: {(role, layer): float32 [rows, cols]} for every projection and the LM head (under
    ROLE_LM_HEAD, or ROLE_TOK_EMB when tied); gains: {(role, layer): float32 vector} for the
    RMSNorm gains (ATTN_NORM, FFN_NORM, ATTN_Q_NORM, ATTN_K_NORM per layer, OUT_NORM at 0);
    embed_row(tok) -> float32 [n_embd], the token's embedding row. Numerics are FloatRef's with
    the weights held in float32 (exact for ternary values times fp16 scales)."""

    def __init__(self, mc, weights, gains, embed_row, kv_fp16=True, dn_tensors=None):
        self.n_layer, self.n_embd = mc.n_layer, mc.n_embd
        self.n_head, self.n_kv, self.hd = mc.n_head, mc.n_kv_head, mc.head_dim
        self.rope_n = mc.rope_dims or mc.head_dim
        self.eps = f32(mc.rms_eps)
        self.gated = bool(mc.attn_gated)
        self.hb, self.hwidths = 0, []
        self.vocab = mc.vocab
        self.dn = [mc.layer_type(l) == "deltanet" for l in range(mc.n_layer)]
        self.nk, self.hk = mc.dn_num_k_heads, mc.dn_k_head_dim
        self.nv, self.hv = mc.dn_num_v_heads, mc.dn_v_head_dim
        self.K = max(mc.dn_conv_kernel, 1)
        # Gated DeltaNet layers: dn_tensors {(role, layer): float32} of SSM_CONV [C, K], SSM_A,
        # SSM_DT, SSM_NORM; their projections (ATTN_QKV, ATTN_ZGATE, SSM_BETA, SSM_ALPHA,
        # SSM_OUT) are in `weights`.
        dn_tensors = dn_tensors or {}
        self.norm_ssm, self.ssm_a, self.ssm_dt, self.conv_w = {}, {}, {}, {}
        for l in range(mc.n_layer):
            if self.dn[l]:
                self.norm_ssm[l] = dn_tensors[(L.ROLE_SSM_NORM, l)]
                self.ssm_a[l] = dn_tensors[(L.ROLE_SSM_A, l)]
                self.ssm_dt[l] = dn_tensors[(L.ROLE_SSM_DT, l)]
                self.conv_w[l] = dn_tensors[(L.ROLE_SSM_CONV, l)].reshape(-1, self.K)
        self.kv_fp16 = kv_fp16
        self.rope_tab = None
        self.rope_freq = np.array([f32(f32(mc.rope_theta) ** f32(-2.0 * i / self.rope_n))
                                   for i in range(self.rope_n // 2)], dtype=f32)
        self.w32 = weights
        self.head_role = L.ROLE_LM_HEAD if (L.ROLE_LM_HEAD, 0) in weights else L.ROLE_TOK_EMB
        self.norm_attn = [gains[(L.ROLE_ATTN_NORM, l)] for l in range(mc.n_layer)]
        self.norm_ffn = [gains[(L.ROLE_FFN_NORM, l)] for l in range(mc.n_layer)]
        self.norm_q = {l: gains[(L.ROLE_ATTN_Q_NORM, l)] for l in range(mc.n_layer) if not self.dn[l]}
        self.norm_k = {l: gains[(L.ROLE_ATTN_K_NORM, l)] for l in range(mc.n_layer) if not self.dn[l]}
        self.out_norm = gains[(L.ROLE_OUT_NORM, 0)]
        self.embed_row = embed_row
        self.reset()

    def proj(self, role, l, x):
        return (self.w32[(role, l)] @ np.asarray(x, dtype=f32)).astype(f32)

    def proj_many(self, role, l, X):
        return (np.asarray(X, dtype=f32) @ self.w32[(role, l)].T).astype(f32)

    def embed(self, tok):
        return np.asarray(self.embed_row(int(tok)), dtype=f32)
