"""Chat rendering and the tokenizer contract of the session host (the caller's side of the
token-id boundary: speccheck/textio.py:1-90, specification/02-tokenization-and-embedding.md §02.1-02.2).

The engine takes token ids. A chat driver renders the conversation to one string, tokenizes it
without adding special tokens (special tokens stay whole and never merge with neighbouring
text, assumption A-11), feeds the ids, and prints generated ids with the special ones masked.

The special-token literals are assembled from pieces: `<|im_start|>` (248045) and `<|think|>`
(248068) look alike in many terminals, and a mistyped literal only shows up as a tokenization
mismatch.
"""
from __future__ import annotations

import json
from pathlib import Path

_LT, _BAR, _GT = "<", "|", ">"


def _special(name: str) -> str:
    return _LT + _BAR + name + _BAR + _GT


IM_START = _special("im_start")        # 248045
IM_END = _special("im_end")            # 248046, also the engine's stop token
THINK_START = _special("think")        # 248068
THINK_END = _special("end")            # 248069
IM_START_ID = 248045
EOS_PRIMARY_ID = 248046
EOS_LEGACY_ID = 248044                 # legacy stop of the torch path (A-10)
THINK_START_ID = 248068
THINK_END_ID = 248069
EOS_IDS = (EOS_PRIMARY_ID, EOS_LEGACY_ID)
# ids a chat front end never prints as their literal text (engine/chat.py MASKED)
MASKED_IDS = (THINK_START_ID, THINK_END_ID, EOS_PRIMARY_ID, EOS_LEGACY_ID, IM_START_ID)


def render_chat(messages, add_generation_prompt: bool = True, thinking: bool = False) -> str:
    """The text-only subset of the checkpoint's chat template (speccheck/textio.py:28-39,
    specification §02.2): every message becomes `<|im_start|>{role}\\n{content}<|im_end|>\\n`,
    concatenated with nothing between; with `add_generation_prompt` the assistant header follows,
    ending in an open thinking block (`thinking`) or an empty, closed one."""
    parts = []
    for m in messages:
        role, content = m["role"], m["content"]
        if not isinstance(role, str) or not isinstance(content, str):
            raise TypeError("render_chat: role and content must be strings (text-only subset)")
        parts += [IM_START, role, "\n", content, IM_END, "\n"]
    if add_generation_prompt:
        parts += [IM_START, "assistant\n", THINK_START, "\n"]
        if not thinking:
            parts += ["\n", THINK_END, "\n\n"]
    return "".join(parts)


def render_continuation(text: str, closed: bool) -> str:
    """The next user turn of a conversation whose earlier turns the engine already holds
    (speccheck/chat.py:106-118): the rendered string is extended, never re-rendered, because the
    generation header's empty thinking block is not what a re-render of that assistant turn
    gives. The assistant turn is closed first unless its generation ended on the stop token
    (`closed`); then the user turn and the thinking-off generation header."""
    head = "" if closed else IM_END + "\n"
    return head + render_chat([{"role": "user", "content": text}])


def render_test_prompt(test: dict, base: Path | None = None) -> str:
    """The prompt of one benchmark test file (testdata/README.md schema 1: `instruction`, then
    the text of `content_file` if it names one), rendered as one user turn with thinking off and
    the generation prompt appended (testdata/index.json `conventions.rendering`)."""
    text = test["instruction"]
    cf = test.get("content_file")
    if cf not in (None, "None", ""):
        text += Path(base or ".", cf).read_text()
    return render_chat([{"role": "user", "content": text}], thinking=False)


class Tokenizer:
    """Tokenize without added specials, decode, and the special ids, over a model directory's
    `tokenizer.json` (speccheck/textio.py:42-76 wraps transformers' AutoTokenizer over the same
    file). The think tokens are resolved from the file's own added-token table by id, never from
    the literals. No tokenizer ships with this build: a caller points it at a checkpoint."""

    def __init__(self, model_dir: str | Path):
        from tokenizers import Tokenizer as _Tok
        path = Path(model_dir)
        if path.is_dir():
            path = path / "tokenizer.json"
        if not path.exists():
            raise FileNotFoundError(f"no tokenizer.json at {path}")
        self.tok = _Tok.from_file(str(path))
        added = {t["id"]: t["content"] for t in json.loads(path.read_text()).get("added_tokens", [])}
        self.think = (added.get(THINK_START_ID), added.get(THINK_END_ID))
        self.added = added

    def encode(self, text: str) -> list[int]:
        return list(self.tok.encode(text, add_special_tokens=False).ids)

    def render_ids(self, messages, thinking: bool = False) -> list[int]:
        return self.encode(render_chat(messages, thinking=thinking))

    def decode(self, ids) -> str:
        return self.tok.decode(list(ids), skip_special_tokens=False)

    def display(self, ids) -> str:
        """Generated ids as text, with every id of MASKED_IDS shown as `[id]` instead of its
        literal (engine/chat.py: a literal end-of-turn token in a transcript ends a message)."""
        out, run = [], []
        for t in ids:
            if int(t) in MASKED_IDS:
                if run:
                    out.append(self.decode(run))
                    run = []
                out.append(f"[{int(t)}]")
            else:
                run.append(int(t))
        if run:
            out.append(self.decode(run))
        return "".join(out)
