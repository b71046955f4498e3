"""Token sampling (firmware/infer.c:385-496): the oracle's restatement on hand-made cases, and the
GPU sampler against it on the logits the GPU decoder produced, step by step."""

import numpy as np
import pytest

from oracle import sampler as S


def test_xorshift32_stream():
    """x ^= x << 13; x ^= x >> 17; x ^= x << 5 (32-bit): from 1, 270369, then 67634689."""
    assert S.xorshift32(1) == 270369
    assert S.xorshift32(270369) == 67634689
    assert all(S.xorshift32(x) != 0 for x in (1, 0x9E3779B9, 0xFFFFFFFF))   # never leaves a nonzero state


def test_candidates_are_slice_maxima():
    rng = np.random.default_rng(0)
    lg = rng.normal(size=1000).astype(np.float32)
    c = S.candidates(lg, 1000, 1)
    assert len(c) == 32 and c[0][1] == int(np.argmax(lg[:32]))       # 32 rows a slice
    assert max(v for v, _ in c) == lg.max()                             # the global best is one
    c2 = S.candidates(lg, 1000, 2)                                      # 500 rows a channel
    toks = [*range(16), *range(500, 516)]                              # slice 0 of both channels
    assert c2[0][1] == toks[int(np.argmax(lg[toks]))]
    assert all(t < 1000 for _, t in c2) and max(v for v, _ in c2) == lg.max()


def test_penalty_temperature_and_top_p():
    cands = [(np.float32(2.0), 7), (np.float32(1.5), 9), (np.float32(-1.0), 3)]
    assert S.pick(cands, [], 0.0, 1.0, 1.0, 5)[0] == 7                  # greedy
    assert S.pick(cands, [7], 0.0, 1.0, 1.5, 5)[0] == 9                 # 2.0 / 1.5 < 1.5
    assert S.pick([(np.float32(-1.0), 3), (np.float32(-1.2), 4)], [3], 0.0, 1.0, 1.5, 5)[0] == 4   # -1 * 1.5
    assert all(S.pick(cands, [], 1.0, 1e-6, 1.0, s)[0] == 7 for s in range(1, 50))   # top_p keeps one
    picks = set()
    rng = 1
    for _ in range(200):
        t, rng = S.pick(cands, [], 5.0, 1.0, 1.0, rng)
        picks.add(t)
    assert picks == {7, 9, 3}


def test_draw_against_closed_forms():
    """The draw of smp_pick (firmware/infer.c:456-466) on cases whose answer is fixed without its
    loop. x is the next xorshift32 state and u = (x >> 8) / 2^24 the uniform it yields.
    * 32 equal candidates, top_p 1: the mass is 32 and the draw picks index floor(32 u) = x >> 27.
    * 4 equal candidates, top_p 0.5: the cut (0.5 * 4 = 2) is reached at the second candidate
      (acc >= cut), so two are kept, the draw is scaled by their mass 2 and picks x >> 31. Scaling
      by the whole mass, cutting one candidate early or late, or a strict acc > cut would each
      pick otherwise for some u in [0.25, 1).
    * Two candidates d apart at temperature T, top_p 1: the second is picked iff
      u * (1 + e^(-d/T)) >= 1."""
    def states(pred, n=12):
        out, s = [], 12345
        while len(out) < n:
            s = S.xorshift32(s)
            if pred(S.xorshift32(s)):
                out.append(s)
        return out

    eq32 = [(np.float32(0.5), 100 + i) for i in range(32)]
    for s in states(lambda x: True, 40):
        x = S.xorshift32(s)
        t, r = S.pick(eq32, [], 0.7, 1.0, 1.0, s)
        assert r == x and t == 100 + (x >> 27)
    eq4 = [(np.float32(1.0), t) for t in (10, 20, 30, 40)]
    for quarter in range(4):
        for s in states(lambda x: x >> 30 == quarter, 5):
            x = S.xorshift32(s)
            assert S.pick(eq4, [], 1.0, 0.5, 1.0, s)[0] == (10, 20)[x >> 31], (quarter, s)
    d, T = 1.0, 0.5
    two = [(np.float32(2.0), 1), (np.float32(2.0 - d), 2)]
    thr = 1.0 / (1.0 + np.exp(-d / T))
    for s in states(lambda x: abs((x >> 8) / 2.0**24 - thr) > 1e-4, 30):
        u = (S.xorshift32(s) >> 8) / 2.0**24
        assert S.pick(two, [], T, 1.0, 1.0, s)[0] == (2 if u >= thr else 1)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid"])
def test_gpu_sampler_matches_the_oracle(tiny_images, golden, name):
    """Generate with sampling on the GPU, then replay the same tokens teacher-forced: each
    generated token is the oracle's pick on the GPU's logits of its position, with the same
    xorshift32 stream and token history."""
    from trixium_amd.model import Decoder
    dec = Decoder.from_image(tiny_images[(name, True)], max_new=32)
    prompt = golden[f"prompt/{name}"]
    temp, top_p, rep, seed = 0.8, 0.9, 1.3, 1234
    dec.set_sampling(temp, top_p, rep, seed)
    dec.reset()
    toks = dec.generate(prompt, 16)
    dec.set_sampling()                                   # greedy again
    dec.reset()
    seq = list(prompt)
    logits = [dec.forward(prompt)]
    for t in toks[:-1]:
        logits.append(dec.forward([t]))
    rng = seed
    for k, lg in enumerate(logits):
        want, rng = S.pick(S.candidates(lg, dec.vocab, 1), seq, temp, top_p, rep, rng)
        assert toks[k] == want, (k, toks[k], want)
        seq.append(toks[k])
    dec.reset()
    greedy = dec.generate(prompt, 8)
    assert greedy == golden[f"fastref_tokens/{name}"][:8]
