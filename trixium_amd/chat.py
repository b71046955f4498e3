"""Chat with a BONS model on the GPU: the host loop of the reference's `trixium chat`
(software/cli.py:217-268 -> software/user/trixium_chat.c), with the decoder in HBM instead of
the FPGA behind a console.

Each user line becomes one chat-template turn (Tokenizer.turn); the reply is generated one token
per forward (the firmware's `genb N stop` contract: no forward after the last token) and streamed
as text until <|im_end|> or the reply cap. The conversation stays in the decoder's context, so a
turn continues the previous one. Sampling follows the firmware's `sample` command
(temperature, top-p, repetition; firmware/infer.c:401-407).

    python -m trixium_amd.chat -m model.bons -z tokenizer.bin [-n 256] [-S T,P,R] [-s SEED]
                               [-y SYSTEM] [-r] [-p PROMPT ...]
"""

import argparse
import sys


class Chat:
    """A conversation: one Decoder, one Tokenizer, the position carried from turn to turn."""

    def __init__(self, decoder, tokenizer, system=None, raw=False, max_reply=256):
        self.dec, self.tok = decoder, tokenizer
        self.system, self.raw, self.max_reply = system, raw, max_reply
        self.first, self.prev_closed = True, True
        self.dec.reset()

    def turn_ids(self, text):
        if self.raw:
            return self.tok.encode(text)
        return self.tok.turn(text, self.system, self.first, self.prev_closed)

    def reply(self, text, out=None):
        """Feed one user turn and generate the reply: (token ids, text). Tokens stream to `out`
        (a file-like) as they decode."""
        ids = self.turn_ids(text)
        room = self.dec.cfg.max_ctx - (self.dec.position() + 1) - len(ids)
        n_max = min(self.max_reply, room)
        if n_max < 1:
            raise ValueError("the conversation has reached the context limit")
        feed = self.tok.stream_decoder()
        got, pieces = [], []
        nxt = ids
        for _ in range(n_max):
            t = self.dec.generate(nxt, 1)[0]
            got.append(t)
            if t == self.tok.im_end and not self.raw:
                break
            s = feed(t)
            pieces.append(s)
            if out is not None and s:
                out.write(s)
                out.flush()
            nxt = [t]
        self.first = False
        # A reply that ended on <|im_end|> left it in the context; a cut one gets it next turn.
        self.prev_closed = bool(got) and got[-1] == self.tok.im_end
        return got, "".join(pieces)


def main(argv=None):
    ap = argparse.ArgumentParser(description="chat with a BONS model on the GPU")
    ap.add_argument("-m", "--image", required=True, help="BONS image")
    ap.add_argument("-z", "--tokenizer", required=True, help="BTOK tokenizer (python -m trixium_amd.tokenizer)")
    ap.add_argument("-n", type=int, default=256, help="reply cap in tokens (a reply ends at <|im_end|> anyway)")
    ap.add_argument("-S", metavar="T,P,R", default=None, help="sample: temperature, top-p, repetition penalty")
    ap.add_argument("-s", type=int, default=0, help="sampling seed (0 keeps the stream)")
    ap.add_argument("-y", "--system", default=None, help="system message of the first turn")
    ap.add_argument("-r", "--raw", action="store_true", help="raw completion: no chat template")
    ap.add_argument("-p", "--prompt", action="append", help="user turns to run instead of reading stdin")
    ap.add_argument("--max-ctx", type=int, default=None)
    a = ap.parse_args(argv)
    from .model import Decoder
    from .tokenizer import Tokenizer
    tok = Tokenizer.from_btok(a.tokenizer)
    dec = Decoder.from_image(a.image, max_ctx=a.max_ctx, max_new=1)
    if a.S:
        t, p, r = (float(v) for v in a.S.split(","))
        dec.set_sampling(t, p, r, seed=a.s)
    chat = Chat(dec, tok, a.system, a.raw, a.n)
    lines = a.prompt if a.prompt else (ln.rstrip("\n") for ln in sys.stdin)
    for line in lines:
        if not line:
            continue
        chat.reply(line, out=sys.stdout)
        sys.stdout.write("\n")
        sys.stdout.flush()
    dec.close()


if __name__ == "__main__":
    main()
