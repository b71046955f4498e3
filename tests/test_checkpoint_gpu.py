"""Decode-state checkpoints (firmware/infer.c:1926-1960 forward_checked, firmware/hybrid.c:2904-2930
hybrid_ckpt_save/restore): forwards run again from a restored checkpoint give the same logits and
tokens bit for bit, also after other forwards moved the KV cache, the DeltaNet state and the
sampler's stream on in between."""

import numpy as np
import pytest

from trixium_amd._lib import TrxError

pytestmark = pytest.mark.gpu


def _decoder(path, **kw):
    from trixium_amd.model import Decoder
    return Decoder.from_image(path, **kw)


def _run(dec, tokens):
    """Logits after each of `tokens` fed one forward at a time."""
    return np.stack([dec.forward([t]) for t in tokens])


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-hybrid"])
@pytest.mark.parametrize("use_graph", [True, False])
def test_forwards_rerun_from_a_checkpoint(tiny_images, golden, name, use_graph):
    prompt = golden[f"prompt/{name}"]
    cont = golden[f"fastref_tokens/{name}"][:12]
    dec = _decoder(tiny_images[(name, True)], use_graph=use_graph)
    dec.reset()
    dec.forward(prompt)
    p0 = dec.position()
    dec.checkpoint()
    first = _run(dec, cont)
    # Other tokens move the state on (KV rows past p0, DeltaNet state, position).
    dec.restore()
    assert dec.position() == p0
    _run(dec, [(t * 7 + 3) % dec.vocab for t in cont[:5]])
    dec.restore()
    assert dec.position() == p0
    again = _run(dec, cont)
    print(f"{name} graph={use_graph}: {len(cont)} forwards from position {p0}, max |diff| "
          f"{float(np.max(np.abs(again - first))):.3g}")
    assert np.array_equal(first, again)
    # The same as an uninterrupted run from a fresh state.
    dec.reset()
    dec.forward(prompt)
    assert np.array_equal(_run(dec, cont), first)


def test_sampled_tokens_repeat_after_restore(tiny_images, golden):
    name = "tiny-hybrid"
    prompt = golden[f"prompt/{name}"]
    dec = _decoder(tiny_images[(name, True)], max_new=16)
    dec.set_sampling(temperature=0.9, top_p=0.95, repetition=1.1, seed=12345)
    dec.reset()
    dec.checkpoint()
    a = dec.generate(prompt, 16)
    dec.restore()
    b = dec.generate(prompt, 16)
    dec.restore()
    dec.generate(prompt[:3], 4)
    dec.restore()
    c = dec.generate(prompt, 16)
    print("sampled:", a)
    assert a == b == c
    assert len(set(a)) > 1


def test_restore_without_a_checkpoint_is_an_error(tiny_images):
    dec = _decoder(tiny_images[("tiny-qwen3", True)])
    with pytest.raises(TrxError):
        dec.restore()


def test_restore_after_a_reset_rewrote_the_rows_is_an_error(tiny_images, golden):
    """The KV rows are not in the checkpoint: forwards after a reset rewrite the rows below the
    checkpoint's position, so its restore is refused."""
    name = "tiny-qwen3"
    prompt = golden[f"prompt/{name}"]
    dec = _decoder(tiny_images[(name, True)])
    dec.reset()
    dec.forward(prompt)
    dec.checkpoint()
    dec.reset()
    dec.forward(prompt[:4])
    with pytest.raises(TrxError):
        dec.restore()


def test_restore_past_the_kv_window_undoes_one_forward(tiny_images, golden):
    """With the KV ring past the window a forward overwrites the ring slot of the position that
    leaves the window: one forward can be run again exactly (the firmware's retry), more are
    refused."""
    name = "tiny-hybrid"
    toks = ((golden[f"prompt/{name}"] + golden[f"fastref_tokens/{name}"]) * 2)[:30]
    dec = _decoder(tiny_images[(name, True)], max_ctx=20)
    dec.set_kv_ring(1, 5)
    dec.reset()
    for t in toks[:26]:
        dec.forward([t])
    dec.checkpoint()
    first = dec.forward([toks[26]])
    dec.restore()
    assert np.array_equal(dec.forward([toks[26]]), first)
    dec.restore()
    dec.forward([toks[26]])
    dec.forward([toks[27]])
    with pytest.raises(TrxError):
        dec.restore()
