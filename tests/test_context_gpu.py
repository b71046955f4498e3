"""The headline shapes at the contexts their workloads run at, against the float oracle.

The bench decodes the Qwen3-8B shape after a 2048-token prompt, the Qwen3-1.7B shape after 512
and the Qwen3.5-27B hybrid after 1024. At those contexts the decode attention splits each kv
head's positions over 32 blocks and a block takes its positions in several passes (5 at 8B and
27B, 2 at 1.7B), the o projection merges 32 splits of many positions, and the prompt runs through
the batched prefill's matrix-core causal attention over the whole prompt. Each test here runs
that configuration on two layers at the full width (every weight from the device generator, read
back from HBM for the oracle; the full LM head): the prompt through the batched prefill, then
decode positions; the oracle (TensorRef with an fp16 KV cache) runs the prompt as one
teacher-forced sequence and the decode positions one by one. Checked: logits at the last prompt
position and at every decode position within 2e-3 of the oracle (relative to the largest logit),
and the greedy ids identical, both stepped and through the graph-replayed generate loop the bench
times. The split count and the passes per split the kernel takes are asserted, so a change of the
attention geometry cannot silently leave the multi-pass paths untested. The 27B hybrid also runs
at eight layers of its layer pattern against the oracle, and at its full 64-layer depth with
size-independent checks.
"""

import math

import numpy as np
import pytest

from test_headline_gpu import _oracle, _oracle_hybrid, _rel_err
from trixium_amd import configs as C, layout as L, synth

pytestmark = pytest.mark.gpu

TRIT5 = L.KIND_TERNARY5


def _passes(dec, T):
    """(splits, passes per split) of the decode attention over T positions."""
    S, ppp = dec.attention_splits
    return S, math.ceil(math.ceil(T / S) / ppp)


def _run(dec, ref, prompt, n_dec, tag):
    """Prompt through the batched prefill (GPU) and as one sequence (oracle), then n_dec greedy
    positions teacher-forced by the oracle's ids; returns the ids."""
    got = dec.forward(prompt)                      # prefill of all but the last token, then a step
    ref.prefill(prompt[:-1])
    want = ref.step(prompt[-1])
    errs, ids = [_rel_err(got, want)], []
    for i in range(n_dec):
        nxt = int(np.argmax(want))
        assert int(np.argmax(got)) == nxt, (tag, i)
        ids.append(nxt)
        if i + 1 < n_dec:
            got = dec.forward([nxt])
            want = ref.step(nxt)
            errs.append(_rel_err(got, want))
    print(f"{tag}: last prompt position rel err {errs[0]:.2e}, decode positions max {max(errs[1:]):.2e}",
          flush=True)
    assert max(errs) <= 2e-3
    return ids


@pytest.mark.timeout(900)
@pytest.mark.parametrize("shape,n_prompt,max_ctx,n_dec,min_passes",
                         [("8b", 2048, 4096, 32, 5), ("1.7b", 512, 1024, 32, 2)])
def test_dense_shape_at_its_context(shape, n_prompt, max_ctx, n_dec, min_passes):
    from trixium_amd.model import Decoder
    base = C.QWEN3_8B if shape == "8b" else C.QWEN3_1P7B
    mc = base.replace(name=base.name + "-2l", n_layer=2, max_ctx=max_ctx)
    seed = 41 if shape == "8b" else 42
    dec = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=n_dec, prefill_chunk=n_prompt)
    assert dec.packed_ops & 31 == 31
    S, npass = _passes(dec, n_prompt + 1)
    print(f"{shape}: {S} splits per kv head, {npass} passes per split at the first decode position", flush=True)
    assert S == 32 and npass >= min_passes
    print(f"{shape}: reading the weights back", flush=True)
    ref = _oracle(dec, mc, seed)
    prompt = synth.random_prompt(mc, n_prompt, seed)
    ids = _run(dec, ref, prompt, n_dec, shape)
    assert dec.generate_fresh(prompt, n_dec) == ids
    dec.close()


@pytest.mark.timeout(900)
def test_hybrid_27b_at_its_context():
    """One Gated DeltaNet and one gated attention layer at the full 27B width (head_dim 256: 8
    positions per pass, 33 per split at 1040 positions): a 1024-token prompt (the DeltaNet state
    and conv window carried over it by the prefill's scan), then 16 decode positions."""
    from trixium_amd.model import Decoder
    n_prompt, n_dec = 1024, 16
    mc = C.QWEN35_27B.replace(name="qwen3.5-27b-shape-2l", n_layer=2, layer_types=("deltanet", "attn"),
                              max_ctx=1152)
    seed = 43
    dec = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=n_dec, prefill_chunk=n_prompt)
    S, npass = _passes(dec, n_prompt + 1)
    print(f"27b: {S} splits per kv head, {npass} passes per split at the first decode position", flush=True)
    assert S == 32 and npass >= 5
    print("27b: reading the weights back", flush=True)
    ref = _oracle_hybrid(dec, mc, seed)
    prompt = synth.random_prompt(mc, n_prompt, seed)
    ids = _run(dec, ref, prompt, n_dec, "27b")
    assert dec.generate_fresh(prompt, n_dec) == ids
    dec.close()


@pytest.mark.timeout(900)
def test_hybrid_27b_eight_layers_match_the_oracle():
    """Eight layers of the 27B hybrid at the full width (the 3 Gated DeltaNet : 1 gated attention
    pattern twice, the full 248320-row head), against the oracle over a 64-token prompt and 8
    decode positions, with the library's kernels and with every projection on the row-packet
    kernel (packed_ops 0, int16 activations)."""
    from trixium_amd.model import Decoder
    mc = C.QWEN35_27B.replace(name="qwen3.5-27b-shape-8l", n_layer=8, max_ctx=128)
    seed = 45
    prompt = synth.random_prompt(mc, 64, seed)
    ids = None
    for packed in (-1, 0):
        dec = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=8, packed_ops=packed, prefill_chunk=64)
        if ids is None:
            print("27b 8 layers: reading the weights back", flush=True)
            ref = _oracle_hybrid(dec, mc, seed)
        ref.reset()
        got = _run(dec, ref, prompt, 8, f"27b 8 layers packed_ops {dec.packed_ops}")
        assert ids is None or got == ids
        ids = got
        dec.close()


@pytest.mark.timeout(900)
def test_hybrid_27b_full_depth_properties():
    """All 64 layers of the 27B hybrid (48 Gated DeltaNet, 16 gated attention): graph replay
    bitwise equal to eager launches, the batched prefill against one position per forward, finite
    logits. (At this depth the random synthetic hybrid amplifies float32 rounding differences
    about ten-thousandfold: the prefill and the one-position forwards, each accurate to float32
    per operation, end 1.5e-3 apart in the logits. Kernels that round differently are therefore
    compared with the oracle at eight layers instead.)"""
    from trixium_amd.model import Decoder
    mc = C.QWEN35_27B.replace(max_ctx=64)
    seed = 44
    prompt = synth.random_prompt(mc, 12, seed)
    a = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=16, use_graph=True)
    la = [a.forward(prompt)] + [a.forward([t]) for t in (5, 77777)]
    assert all(np.isfinite(v).all() for v in la)
    a.reset()
    ta = a.generate(prompt, 8)
    a.reset()
    lb = [a.forward(prompt, use_graph=False)] + [a.forward([t], use_graph=False) for t in (5, 77777)]
    for x, y in zip(la, lb):
        assert np.array_equal(x, y)
    a.reset()
    assert a.generate(prompt, 8, use_graph=False) == ta
    a.close()
    p = Decoder.synthetic(mc, seed, weight_kind=TRIT5, max_new=16, prefill_chunk=8)
    lp = p.forward(prompt)
    print(f"27b full depth: prefill vs one position per forward rel err {_rel_err(lp, la[0]):.2e}", flush=True)
    assert np.isfinite(lp).all() and _rel_err(lp, la[0]) <= 1e-2
    p.close()
