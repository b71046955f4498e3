"""Byte-level BPE tokenizer for the chat loop: the BTOK export of a HuggingFace tokenizer.json
(model/tokenizer.py's format) and an encoder/decoder over it.

BTOK v2 (model/tokenizer.py:10-16,99-111; the file format the reference's C tool and firmware
read, kept byte for byte):
    "BTOK", u32 version = 2, u32 n_vocab, u32 n_merges, 32-byte SHA-256 of the tokenizer.json,
    n_vocab x {u32 len, the token's raw bytes}   (token id order; added tokens as UTF-8)
    n_merges x {u32 a, u32 b, u32 a+b}           (rank order = merge priority)

The encoder splits text with the Qwen / GPT-2 pre-tokenizer pattern (with true Unicode letter
and number classes, after NFC normalization, as the HuggingFace tokenizer does), then merges each
piece's bytes by rank. A chat turn adds the template's special tokens by id
(software/lib/trixium_tok.c:303-334 ttok_turn).
"""

import codecs
import hashlib
import json
import os
import struct
import unicodedata

import regex

# The Qwen2/Qwen3 pre-tokenizer split.
PRETOKENIZE = regex.compile(r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}"
                            r"| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")

# Reference prompts whose encodings check an encoder against the source tokenizer
# (model/tokenizer.py:47-56).
TEST_PROMPTS = [
    "The capital of France is",
    "Hello world!",
    "def fibonacci(n):",
    "1234 + 5678 = ",
    "  leading spaces and\ttabs\n",
    "Emoji: \U0001F600 and accents: café naïve",
    "A" * 40,
    "The quick brown fox jumps over the lazy dog. It was 2026, and the FK33 ran at 200 MHz.",
]


def byte_to_unicode():
    """GPT-2's byte -> printable character map (the alphabet tokenizer.json stores tokens in):
    printable Latin-1 bytes map to themselves, the other 68 to code points 256, 257, ..."""
    keep = [*range(0x21, 0x7F), *range(0xA1, 0xAD), *range(0xAE, 0x100)]
    out, extra = {}, 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + extra)
            extra += 1
    return out


def export_tokenizer(tokenizer_json, out, tests=None):
    """tokenizer.json (BPE) -> BTOK file `out`, plus reference encodings of TEST_PROMPTS
    (tokenizer_tests.txt next to `out`, or `tests`) when the `tokenizers` package is present."""
    with open(tokenizer_json, "rb") as f:
        raw = f.read()
    d = json.loads(raw.decode("utf-8"))
    model = d["model"]
    if model.get("type") != "BPE":
        raise ValueError(f"unsupported tokenizer type {model.get('type')}")
    u2b = {c: b for b, c in byte_to_unicode().items()}

    def token_bytes(tok):
        try:
            return bytes(u2b[c] for c in tok)
        except KeyError:
            return tok.encode("utf-8")          # outside the byte alphabet: literal UTF-8

    vocab = model["vocab"]
    added = d.get("added_tokens", [])
    # Added tokens can sit above the BPE vocabulary (Qwen3: 151643..151668): size by both.
    n_vocab = max([max(vocab.values())] + [a["id"] for a in added]) + 1
    toks = [b""] * n_vocab
    for tok, tid in vocab.items():
        toks[tid] = token_bytes(tok)
    for a in added:
        toks[a["id"]] = a["content"].encode("utf-8")
    merges = []
    for m in model.get("merges", []):
        a, b = m.split(" ", 1) if isinstance(m, str) else (m[0], m[1])
        ia, ib, iab = vocab.get(a), vocab.get(b), vocab.get(a + b)
        if ia is not None and ib is not None and iab is not None:
            merges.append((ia, ib, iab))
    with open(out, "wb") as f:
        f.write(b"BTOK" + struct.pack("<III", 2, n_vocab, len(merges)) + hashlib.sha256(raw).digest())
        for t in toks:
            f.write(struct.pack("<I", len(t)) + t)
        for m in merges:
            f.write(struct.pack("<III", *m))
    tests = tests or os.path.join(os.path.dirname(os.path.abspath(out)), "tokenizer_tests.txt")
    try:
        from tokenizers import Tokenizer as HFTokenizer
    except ImportError:
        return n_vocab, len(merges)
    hf = HFTokenizer.from_file(tokenizer_json)
    with open(tests, "w", encoding="utf-8") as f:
        for p in TEST_PROMPTS:
            f.write(json.dumps(p) + "\t" + " ".join(str(i) for i in hf.encode(p, add_special_tokens=False).ids) + "\n")
    return n_vocab, len(merges)


class Tokenizer:
    """Encoder and decoder over a BTOK file."""

    def __init__(self, tokens, merges, sha256=b""):
        self.tokens = tokens                        # id -> raw bytes
        self.sha256 = sha256
        self.ranks = {(a, b): (r, ab) for r, (a, b, ab) in enumerate(merges)}
        self.byte_id = {}
        for i, t in enumerate(tokens):
            if len(t) == 1 and t[0] not in self.byte_id:
                self.byte_id[t[0]] = i
        find = {t: i for i, t in enumerate(tokens) if t}
        self.im_start = find.get(b"<|im_start|>", -1)
        self.im_end = find.get(b"<|im_end|>", -1)
        self.think = find.get(b"<think>", -1)
        self.think_end = find.get(b"</think>", -1)

    @classmethod
    def from_btok(cls, path):
        with open(path, "rb") as f:
            data = f.read()
        if data[:4] != b"BTOK":
            raise ValueError(f"{path}: not a BTOK tokenizer")
        version, n_vocab, n_merges = struct.unpack_from("<III", data, 4)
        if version != 2:
            raise ValueError(f"{path}: BTOK version {version} (2 expected)")
        sha, off = data[16:48], 48
        tokens = []
        for _ in range(n_vocab):
            (n,) = struct.unpack_from("<I", data, off)
            tokens.append(data[off + 4:off + 4 + n])
            off += 4 + n
        merges = [struct.unpack_from("<III", data, off + 12 * i) for i in range(n_merges)]
        if off + 12 * n_merges != len(data):
            raise ValueError(f"{path}: {len(data) - off - 12 * n_merges} trailing bytes")
        return cls(tokens, merges, sha)

    def _bpe(self, piece):
        ids = [self.byte_id[b] for b in piece if b in self.byte_id]
        while len(ids) > 1:
            best = None
            for i in range(len(ids) - 1):
                m = self.ranks.get((ids[i], ids[i + 1]))
                if m is not None and (best is None or m[0] < best[0]):
                    best = (m[0], i, m[1])
            if best is None:
                break
            _, i, res = best
            ids[i:i + 2] = [res]
        return ids

    def encode(self, text):
        """Token ids of `text` (no special tokens parsed out of it)."""
        out = []
        for piece in PRETOKENIZE.findall(unicodedata.normalize("NFC", text)):
            out.extend(self._bpe(piece.encode("utf-8")))
        return out

    def piece(self, i):
        """The raw bytes of token i (none for an id outside the vocabulary: a model's vocabulary
        can be padded past the tokenizer's)."""
        return self.tokens[i] if 0 <= i < len(self.tokens) else b""

    def decode(self, ids):
        return b"".join(self.piece(i) for i in ids).decode("utf-8", errors="replace")

    def stream_decoder(self):
        """An incremental decoder: feed(id) -> the text that became complete (UTF-8 sequences
        split over tokens are held back)."""
        dec = codecs.getincrementaldecoder("utf-8")(errors="replace")

        def feed(i):
            return dec.decode(self.piece(i))
        return feed

    def turn(self, text, system=None, first=True, prev_closed=True):
        """One user turn in the Qwen3 chat template, ready for the assistant's reply
        (software/lib/trixium_tok.c:303-334): the previous reply closed (when it was cut) and a
        newline on a continuing conversation; the system message on the first turn; the user
        message; the assistant header; an empty think block when the vocabulary has one. Without
        template tokens, the text alone."""
        if self.im_start < 0 or self.im_end < 0:
            return self.encode(text)
        ids = []
        if not first:
            if not prev_closed:
                ids.append(self.im_end)
            ids += self.encode("\n")
        if first and system:
            ids += [self.im_start] + self.encode("system\n") + self.encode(system) + [self.im_end]
            ids += self.encode("\n")
        ids += [self.im_start] + self.encode("user\n") + self.encode(text) + [self.im_end] + self.encode("\n")
        ids += [self.im_start] + self.encode("assistant\n")
        if self.think >= 0 and self.think_end >= 0:
            ids += [self.think] + self.encode("\n\n") + [self.think_end] + self.encode("\n\n")
        return ids


def main(argv=None):
    import argparse
    ap = argparse.ArgumentParser(description="tokenizer.json -> BTOK (the chat loop's tokenizer)")
    ap.add_argument("tokenizer_json")
    ap.add_argument("out", nargs="?", help="default: tokenizer.bin next to the input")
    a = ap.parse_args(argv)
    out = a.out or os.path.join(os.path.dirname(os.path.abspath(a.tokenizer_json)), "tokenizer.bin")
    n_vocab, n_merges = export_tokenizer(a.tokenizer_json, out)
    print(f"{out}: {n_vocab} tokens, {n_merges} merges")


if __name__ == "__main__":
    main()
