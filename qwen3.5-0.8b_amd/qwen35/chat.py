"""Text chat over the resident session (engine/chat.py and speccheck/chat.py:97-160 drive
`decode_run --session` the same way): each user line is rendered, tokenized without added
specials, fed, and answered by greedy generation up to the stop token or `--max-new`.

    python -m qwen35.chat --model DIR [--max-new 256] [--mtp-k 2] [--thinking]

DIR holds the checkpoint's .safetensors file and its tokenizer.json. The first turn renders the
whole conversation; later turns extend what the lane holds (textio.render_continuation).
Special ids are printed as `[id]`.
"""
from __future__ import annotations

import argparse
import sys

from .engine import Engine
from .session import DEFAULT_CAP, STOP_TOKEN, Session
from .textio import Tokenizer, render_chat, render_continuation


class ChatDriver:
    """One conversation on one Session: `turn(text)` returns the generated ids of the reply."""

    def __init__(self, session: Session, tok: Tokenizer, thinking: bool = False):
        self.s, self.tok, self.thinking = session, tok, thinking
        self.turns = 0
        self.closed = True
        self.log: list[str] = []

    def _run(self, line: str) -> list[str]:
        out: list[str] = []
        self.s.handle(line, out.append)
        self.log += out
        err = [x for x in out if x.startswith("ERROR")]
        if err:
            raise RuntimeError(err[0])
        return out

    def prompt_ids(self, text: str) -> list[int]:
        if self.turns == 0:
            return self.tok.encode(render_chat([{"role": "user", "content": text}], thinking=self.thinking))
        return self.tok.encode(render_continuation(text, self.closed))

    def turn(self, text: str, max_new: int = 256) -> list[int]:
        ids = self.prompt_ids(text)
        if self.turns == 0 and self.s.sampled >= 0:
            raise RuntimeError("the session already holds a conversation: reset it first")
        self._run("feed " + " ".join(str(i) for i in ids))
        gen = [int(x.split()[1]) for x in self._run(f"gen {max_new}") if x.startswith("GEN ")]
        self.turns += 1
        self.closed = bool(gen) and gen[-1] == STOP_TOKEN
        return gen

    def reset(self):
        self._run("reset")
        self.turns, self.closed = 0, True


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="text chat over the MI355X engine")
    ap.add_argument("--model", required=True, help="directory with the .safetensors checkpoint and tokenizer.json")
    ap.add_argument("--cap", type=int, default=DEFAULT_CAP)
    ap.add_argument("--max-new", type=int, default=256)
    ap.add_argument("--mtp-k", type=int, default=2)
    ap.add_argument("--thinking", action="store_true", help="open the thinking block in the first turn")
    a = ap.parse_args(argv)
    tok = Tokenizer(a.model)
    eng = Engine(max_rows=512, max_ctx=a.cap, seed=None)
    eng.load_checkpoint(a.model)
    s = Session(eng, a.cap, mtp_k=a.mtp_k)
    d = ChatDriver(s, tok, a.thinking)
    try:
        for line in sys.stdin:
            line = line.rstrip("\n")
            if line == "/reset":
                d.reset()
                print("[reset]", flush=True)
                continue
            print(tok.display(d.turn(line, a.max_new)), flush=True)
    finally:
        s.close()
        eng.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
