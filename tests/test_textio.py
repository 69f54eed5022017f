"""Chat rendering and the tokenizer contract (speccheck/textio.py:28-76,
specification/02-tokenization-and-embedding.md §02.2). CPU only.

Known answers: the renderings below are written out from §02.2's template (one user turn,
`PING`, thinking off and on), the special ids from its §02.1 table. The tokenizer test builds
a small word-level `tokenizer.json` carrying the model's special ids, since no tokenizer ships
with the reference (it loads the absent checkpoint's, speccheck/textio.py:49-51).
"""
from __future__ import annotations

import json

import pytest

from qwen35 import textio as T

LT, BAR, GT = "<", "|", ">"


def sp(name):
    return LT + BAR + name + BAR + GT


PING_OFF = (sp("im_start") + "user\nPING" + sp("im_end") + "\n" + sp("im_start") + "assistant\n"
            + sp("think") + "\n\n" + sp("end") + "\n\n")
PING_ON = (sp("im_start") + "user\nPING" + sp("im_end") + "\n" + sp("im_start") + "assistant\n"
           + sp("think") + "\n")


def test_render_known_answers():
    msg = [{"role": "user", "content": "PING"}]
    assert T.render_chat(msg) == PING_OFF
    assert T.render_chat(msg, thinking=True) == PING_ON
    assert T.render_chat(msg, add_generation_prompt=False) == sp("im_start") + "user\nPING" + sp("im_end") + "\n"
    assert T.render_chat([], add_generation_prompt=False) == ""


def test_render_multi_turn_concatenates_without_separators():
    msgs = [{"role": "system", "content": "be brief"}, {"role": "user", "content": "a\nb"},
            {"role": "assistant", "content": ""}, {"role": "user", "content": "c"}]
    body = "".join(sp("im_start") + m["role"] + "\n" + m["content"] + sp("im_end") + "\n" for m in msgs)
    assert T.render_chat(msgs, add_generation_prompt=False) == body
    assert T.render_chat(msgs) == body + PING_OFF[len(sp("im_start") + "user\nPING" + sp("im_end") + "\n"):]
    with pytest.raises(TypeError):
        T.render_chat([{"role": "user", "content": ["image"]}])


def test_special_literals_are_distinct():
    assert T.IM_START == sp("im_start") and T.THINK_START == sp("think")
    assert T.IM_START != T.THINK_START and T.IM_END != T.THINK_END
    assert T.EOS_IDS == (248046, 248044)
    assert set(T.MASKED_IDS) == {248045, 248046, 248044, 248068, 248069}


def test_render_test_prompt(tmp_path):
    (tmp_path / "doc.txt").write_text("body text")
    t = {"instruction": "Summarize:\n\n", "content_file": "doc.txt"}
    assert T.render_test_prompt(t, tmp_path) == T.render_chat([{"role": "user", "content": "Summarize:\n\nbody text"}])
    assert T.render_test_prompt({"instruction": "PING", "content_file": None}) == PING_OFF


def _write_tokenizer(path):
    specials = [(T.IM_START, 248045), (T.IM_END, 248046), (T.THINK_START, 248068), (T.THINK_END, 248069),
                (sp("endoftext"), 248044)]
    vocab = {"[UNK]": 0, "user": 1, "assistant": 2, "PING": 3, "\n": 4, "hello": 5}
    vocab.update(dict(specials))
    doc = {"version": "1.0", "truncation": None, "padding": None,
           "added_tokens": [{"id": i, "content": s, "single_word": False, "lstrip": False, "rstrip": False,
                             "normalized": False, "special": True} for s, i in specials],
           "normalizer": None,
           "pre_tokenizer": {"type": "Split", "pattern": {"String": "\n"}, "behavior": "Isolated", "invert": False},
           "post_processor": None, "decoder": None,
           "model": {"type": "WordLevel", "vocab": vocab, "unk_token": "[UNK]"}}
    path.write_text(json.dumps(doc))


def test_tokenizer_keeps_specials_whole(tmp_path):
    pytest.importorskip("tokenizers")
    _write_tokenizer(tmp_path / "tokenizer.json")
    tok = T.Tokenizer(tmp_path)
    ids = tok.render_ids([{"role": "user", "content": "PING"}])
    # every special token is one id, never merged with the text beside it (A-11)
    assert ids == [248045, 1, 4, 3, 248046, 4, 248045, 2, 4, 248068, 4, 4, 248069, 4, 4]
    assert tok.render_ids([{"role": "user", "content": "PING"}], thinking=True) == ids[:10] + [4]
    assert tok.think == (T.THINK_START, T.THINK_END)
    assert tok.display([5, 248046, 3, 248068]) == "hello[248046]PING[248068]"
    with pytest.raises(FileNotFoundError):
        T.Tokenizer(tmp_path / "missing")


def test_continuation_extends_the_rendering():
    first = T.render_chat([{"role": "user", "content": "PING"}])
    # a turn that ended on the stop token already holds the im_end; a truncated one does not
    assert T.render_continuation("PING", closed=True) == PING_OFF
    assert T.render_continuation("PING", closed=False) == sp("im_end") + "\n" + PING_OFF
    assert (first + "reply" + sp("im_end") + T.render_continuation("x", closed=True)).startswith(first)
