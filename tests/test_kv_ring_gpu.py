"""The KV ring past the window (firmware/hybrid.c:156-181,2483): forwards past max_ctx keep the
first `pin` positions and a ring of the most recent ones, against the oracle's ring, whose own
test pins it against attention over exactly those positions. The window is small (20 slots) so
that the decode wraps it twice; every position's logits are compared."""

import numpy as np
import pytest

from oracle.floatref import FloatRef
from trixium_amd import bons
from trixium_amd._lib import TrxError

pytestmark = pytest.mark.gpu

LOGIT_RTOL = 1e-2
CAP, PIN = 20, 5


def _decoder(path, **kw):
    from trixium_amd.model import Decoder
    return Decoder.from_image(path, **kw)


def _tokens(golden, name, n=58):
    return ((golden[f"prompt/{name}"] + golden[f"fastref_tokens/{name}"]) * 3)[:n]


def _rel_err(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / np.max(np.abs(ref)))


def _oracle(path):
    ref = FloatRef(bons.BONSReader(path), kv_fp16=True)
    ref.set_kv_ring(CAP, PIN)
    ref.reset()
    return ref


@pytest.mark.parametrize("name", ["tiny-hybrid", "tiny-qwen3"])
@pytest.mark.parametrize("packed", [-1, 0])
@pytest.mark.parametrize("use_graph", [True, False])
def test_ring_logits_match_the_oracle(tiny_images, golden, name, packed, use_graph):
    path = tiny_images[(name, True)]
    dec = _decoder(path, max_ctx=CAP, packed_ops=packed, use_graph=use_graph)
    dec.set_kv_ring(1, PIN)
    dec.reset()
    assert dec.kv_pin == PIN
    ref = _oracle(path)
    worst = 0.0
    for i, t in enumerate(_tokens(golden, name)):
        err = _rel_err(dec.forward([t]), ref.step(t))
        worst = max(worst, err)
        assert err <= LOGIT_RTOL, (name, i, err)
    print(f"{name} packed={packed} graph={use_graph}: 58 positions through a {CAP}-slot window, "
          f"worst rel err {worst:.2e}")
    assert dec.position() == 57


def test_ring_greedy_tokens_match_the_oracle(tiny_images, golden):
    name = "tiny-hybrid"
    path = tiny_images[(name, True)]
    prompt = golden[f"prompt/{name}"]
    dec = _decoder(path, max_ctx=CAP, max_new=48)
    assert dec.kv_pin == 4                         # a hybrid's default: the ring with the 4 sinks
    dec.set_kv_ring(1, PIN)
    got = dec.generate_fresh(prompt, 48)
    ref = FloatRef(bons.BONSReader(path), kv_fp16=True)
    ref.set_kv_ring(CAP, PIN)
    ref.reset()
    want = ref.generate(prompt, 48)
    print("ring greedy:", got)
    assert got == want


def test_prefill_past_the_window_steps_the_rest(tiny_images, golden):
    """A batched prefill that reaches past the window runs its positions up to max_ctx as a
    chunk and steps the others one forward each."""
    name = "tiny-hybrid"
    path = tiny_images[(name, True)]
    toks = _tokens(golden, name, 32)
    dec = _decoder(path, max_ctx=CAP, prefill_chunk=8)
    dec.set_kv_ring(1, PIN)
    dec.reset()
    ref = _oracle(path)
    a = dec.forward(toks[:16])
    b = dec.forward(toks[16:])
    ra = ref.forward(toks[:16])
    rb = ref.forward(toks[16:])
    assert _rel_err(a, ra) <= LOGIT_RTOL and _rel_err(b, rb) <= LOGIT_RTOL
    assert dec.position() == 31


def test_ring_off_stops_at_the_window(tiny_images, golden):
    name = "tiny-hybrid"
    dec = _decoder(tiny_images[(name, True)], max_ctx=CAP, max_new=8)
    dec.set_kv_ring(0)
    dec.reset()
    assert dec.kv_pin == 0
    dec.forward(_tokens(golden, name, CAP))
    with pytest.raises(TrxError):
        dec.forward([1])
    qwen = _decoder(tiny_images[("tiny-qwen3", True)], max_ctx=CAP)
    assert qwen.kv_pin == 0                        # plain Qwen3 stops at the window by default
