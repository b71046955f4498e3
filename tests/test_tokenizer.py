"""The chat loop's tokenizer: BTOK export (model/tokenizer.py's format) and the encoder against
the HuggingFace tokenizer it was exported from, on a small byte-level BPE trained here with the
Qwen pre-tokenizer (no real tokenizer.json is available offline)."""

import json
import os
import struct

import numpy as np
import pytest

from trixium_amd import tokenizer as T

SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<think>", "</think>"]
TEXT = ["The capital of France is Paris. Hello world! def fibonacci(n): return n if n < 2 else fib(n-1)",
        "café naïve 1234 + 5678 = 6912, ΕΛΛΑΔΑ и Россия, 東京 and 😀 emoji's aren't we'll",
        "The quick brown fox jumps over the lazy dog.\n\n  indented\ttabs   and spaces  \r\n end"] * 40


@pytest.fixture(scope="module")
def hf_json(tmp_path_factory):
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import Regex, Tokenizer, decoders, models, normalizers, pre_tokenizers, trainers
    tk = Tokenizer(models.BPE())
    tk.normalizer = normalizers.NFC()
    tk.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(T.PRETOKENIZE.pattern), behavior="isolated", invert=False),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tk.decoder = decoders.ByteLevel()
    tk.train_from_iterator(TEXT, trainers.BpeTrainer(vocab_size=800, initial_alphabet=pre_tokenizers.ByteLevel.alphabet()))
    tk.add_special_tokens(SPECIALS)          # added tokens above the BPE vocabulary, as Qwen3's
    p = str(tmp_path_factory.mktemp("tok") / "tokenizer.json")
    tk.save(p)
    return p


def test_byte_alphabet_is_gpt2s():
    m = T.byte_to_unicode()
    assert len(set(m.values())) == 256
    assert m[ord("A")] == "A" and m[0x20] == "Ġ" and m[0x0A] == "Ċ" and m[0xAD] == "Ń"


def test_btok_file_layout(hf_json, tmp_path):
    out = str(tmp_path / "tokenizer.bin")
    n_vocab, n_merges = T.export_tokenizer(hf_json, out)
    data = open(out, "rb").read()
    assert data[:4] == b"BTOK" and struct.unpack_from("<III", data, 4) == (2, n_vocab, n_merges)
    import hashlib
    assert data[16:48] == hashlib.sha256(open(hf_json, "rb").read()).digest()
    d = json.load(open(hf_json, encoding="utf-8"))
    assert n_vocab == max(max(d["model"]["vocab"].values()), max(a["id"] for a in d["added_tokens"])) + 1
    tok = T.Tokenizer.from_btok(out)
    assert tok.tokens[tok.im_start] == b"<|im_start|>" and tok.im_start > max(d["model"]["vocab"].values())
    assert os.path.exists(str(tmp_path / "tokenizer_tests.txt"))


def test_encoder_matches_huggingface(hf_json, tmp_path):
    from tokenizers import Tokenizer as HF
    out = str(tmp_path / "tokenizer.bin")
    T.export_tokenizer(hf_json, out)
    tok, hf = T.Tokenizer.from_btok(out), HF.from_file(hf_json)
    prompts = T.TEST_PROMPTS + [t[:120] for t in TEXT[:3]] + ["", " ", "a\n\n\nb", "x' 's 'LL 're", "é" * 30,
                                                            "1234567", "mixed😀😀text", "é decomposed"]
    for p in prompts:
        assert tok.encode(p) == hf.encode(p, add_special_tokens=False).ids, p
        assert tok.decode(tok.encode(p)) == hf.decode(hf.encode(p, add_special_tokens=False).ids)
    # The reference's check file: the same ids as the live encoder.
    for line in open(str(tmp_path / "tokenizer_tests.txt"), encoding="utf-8"):
        p, ids = line.rstrip("\n").split("\t")
        assert tok.encode(json.loads(p)) == [int(i) for i in ids.split()]


def test_chat_turn_template(hf_json, tmp_path):
    """The turn ids equal the HuggingFace encoding of the Qwen3 template text with its special
    tokens (software/lib/trixium_tok.c:303-334)."""
    from tokenizers import Tokenizer as HF
    out = str(tmp_path / "tokenizer.bin")
    T.export_tokenizer(hf_json, out)
    tok, hf = T.Tokenizer.from_btok(out), HF.from_file(hf_json)
    enc = lambda s: hf.encode(s, add_special_tokens=True).ids
    want = enc("<|im_start|>system\nBe brief.<|im_end|>\n<|im_start|>user\nHello world!<|im_end|>\n"
               "<|im_start|>assistant\n<think>\n\n</think>\n\n")
    assert tok.turn("Hello world!", "Be brief.", first=True) == want
    cont = enc("<|im_end|>\n<|im_start|>user\nAnd France?<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n")
    assert tok.turn("And France?", None, first=False, prev_closed=False) == cont
    assert tok.turn("And France?", None, first=False, prev_closed=True) == cont[1:]


def test_stream_decoder_holds_split_utf8(hf_json, tmp_path):
    out = str(tmp_path / "tokenizer.bin")
    T.export_tokenizer(hf_json, out)
    tok = T.Tokenizer.from_btok(out)
    text = "東京 😀 café"
    feed = tok.stream_decoder()
    assert "".join(feed(i) for i in tok.encode(text)) == text


@pytest.mark.gpu
def test_chat_loop_on_the_gpu(hf_json, tmp_path, tiny_images):
    """Two chat turns with the tiny Qwen3 model: each reply is the decoder's greedy continuation
    of the conversation so far (one forward per token, the context carried between turns), as
    one generate over the same ids computes it."""
    from trixium_amd.chat import Chat
    from trixium_amd.model import Decoder
    out = str(tmp_path / "tokenizer.bin")
    T.export_tokenizer(hf_json, out)
    tok = T.Tokenizer.from_btok(out)
    dec = Decoder.from_image(tiny_images[("tiny-qwen3", True)], max_new=1)
    chat = Chat(dec, tok, system="Be brief.", max_reply=6)
    t1 = chat.turn_ids("Hello world!")
    r1, _ = chat.reply("Hello world!")
    t2 = chat.turn_ids("And France?")
    r2, text2 = chat.reply("And France?")
    ref = Decoder.from_image(tiny_images[("tiny-qwen3", True)], max_new=16)
    assert ref.generate_fresh(t1, len(r1)) == r1
    ref.reset()
    assert ref.generate(t1 + r1 + t2, len(r2)) == r2
    assert isinstance(text2, str)
