"""The firmware's token sampler restated in numpy float32 (test infrastructure only, see
oracle/__init__.py). firmware/infer.c:1458-1496 forms the candidates (the head as 32 row-range
ops, one (value, token) per range over every channel's shard of the vocabulary), and
firmware/infer.c:395-466 (smp_pick) picks among them: repetition penalty over the last 64
tokens, temperature, top-p, one xorshift32 draw."""

import numpy as np

f32 = np.float32
SLICES = 32


def xorshift32(x):
    x ^= (x << 13) & 0xFFFFFFFF
    x ^= x >> 17
    x ^= (x << 5) & 0xFFFFFFFF
    return x & 0xFFFFFFFF


def candidates(logits, vocab, n_ch):
    """[(value, token)] in slice order: slice k holds rows r0..r0+rows-1 of every channel's shard
    (rpc = ceil(vocab / n_ch) rows a channel), its first maximum in channel-major order."""
    rpc = -(-vocab // n_ch)
    srows = -(-rpc // SLICES)
    out = []
    for r0 in range(0, rpc, srows):
        rows = min(srows, rpc - r0)
        toks = [c * rpc + r0 + i for c in range(n_ch) for i in range(rows)]
        toks = [t for t in toks if t < vocab]
        if toks:
            vals = np.asarray(logits, f32)[toks]
            j = int(np.argmax(vals))
            out.append((f32(vals[j]), toks[j]))
    return out


def pick(cands, recent, temperature, top_p, repetition, rng, window=64):
    """(token, rng) of smp_pick over `cands` with the token history `recent` (oldest first)."""
    seen = set(recent[-window:]) if window else set()
    lg, tk = [], []
    for v, t in cands:
        v = f32(v)
        if repetition > 1.0 and t in seen:
            v = f32(v / f32(repetition)) if v > 0 else f32(v * f32(repetition))
        lg.append(v)
        tk.append(t)
    best = 0
    for i in range(len(lg)):
        if lg[i] > lg[best]:
            best = i
    if temperature <= 0.0:
        return tk[best], rng
    order = sorted(range(len(lg)), key=lambda i: -lg[i])          # stable, descending
    p = [f32(np.exp(f32(f32(lg[o] - lg[order[0]]) / f32(temperature)))) for o in order]
    total = f32(0)
    for v in p:
        total = f32(total + v)
    cut = f32(f32(top_p) * total)
    acc, keep = f32(0), len(p)
    for i, v in enumerate(p):
        acc = f32(acc + v)
        if acc >= cut:
            keep = i + 1
            break
    rng = xorshift32(rng)
    r = f32(f32(f32(rng >> 8) * f32(1.0 / 16777216.0)) * acc)
    c = f32(0)
    for i in range(keep):
        c = f32(c + p[i])
        if r < c:
            return tk[order[i]], rng
    return tk[order[keep - 1]], rng
