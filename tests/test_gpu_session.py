"""The resident session protocol (decode_run --session, engine/decode_run.cpp:1760-1790,
2436-2680) over the engine: replies and their order, greedy tokens identical to a plain
Forward over the same transcript across turns (the pending-sample rule: a budget-ended turn
drops its unshown sample, the next feed carries only the caller's ids), argument errors that
do not poison, an engine error that poisons until `reset`, the opt-in logits dump, and the
stdin/stdout entry point in a child process."""
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def eng():
    from qwen35 import Engine
    e = Engine(max_rows=64, max_ctx=512, seed=0, use_graph=True)
    yield e
    e.close()


def test_session_turns_match_forward(eng, tmp_path):
    from oracle.weights import lane_prompt_ids
    from qwen35 import Forward, State
    from qwen35.session import Session
    out = []
    s = Session(eng, 512, str(tmp_path))
    emit = out.append
    assert s.ready_line() == "READY cap=512"
    ids1 = [int(t) for t in lane_prompt_ids(9, 0, 12)]
    ids2 = [int(t) for t in lane_prompt_ids(9, 1, 5)]

    s.handle("gen 3", emit)
    assert out[-1].startswith("ERROR gen with no sampled token")
    s.handle("feed " + " ".join(map(str, ids1)), emit)
    assert out[-1] == f"FED n=12 prefix_len=12"
    n0 = len(out)
    s.handle("dump 14", emit)
    assert out[-1] == f"DUMP armed=1 min=14 max=14 dir={tmp_path}"
    s.handle("gen 5", emit)
    lines = out[n0 + 1:]
    gens = [l for l in lines if l.startswith("GEN ")]
    assert [int(l.split()[2]) for l in gens] == [11, 12, 13, 14, 15]
    toks = [int(l.split()[1]) for l in gens]
    assert lines[-1] == "END steps=5 stop=0 prefix_len=17"
    dumps = [l for l in lines if l.startswith("DUMP seq=")]
    assert len(dumps) == 1 and " kind=step pos=14 " in dumps[0]
    row = np.fromfile(tmp_path / dumps[0].split("file=")[1], dtype=np.float32)
    assert row.size == 248320 and int(np.argmax(row)) == toks[3]   # the row at 14 decides "GEN <id> 14"
    s.handle("dump off", emit)
    assert out[-1] == "DUMP armed=0 written=1"

    ref = Forward(eng, State(eng, 1, 512)).greedy(ids1, 4, stop_on_eos=False)
    assert toks == ref[:5]

    s.handle("gen 1", emit)                   # the budget-ended turn left no pending sample
    assert out[-1].startswith("ERROR gen with no sampled token")
    s.handle("feed " + " ".join(map(str, ids2)), emit)
    assert out[-1] == "FED n=5 prefix_len=22"
    s.handle("gen 3", emit)
    toks2 = [int(l.split()[1]) for l in out[-4:-1]]
    assert out[-1] == "END steps=3 stop=0 prefix_len=25"
    ref2 = Forward(eng, State(eng, 1, 512)).greedy(ids1 + toks + ids2, 2, stop_on_eos=False)
    assert toks2 == ref2[:3]
    s.handle("stats", emit)
    assert out[-1] == "PREFIX p=25 sampled=-1 stopped=0"

    s.handle("gen x", emit)
    s.handle("feed 1 2", emit)                # argument errors above did not poison
    assert out[-1] == "FED n=2 prefix_len=27"
    s.handle("feed 999999999", emit)          # out-of-range id: the engine refuses -> poisoned
    assert out[-1].startswith("ERROR ")
    s.handle("gen 1", emit)
    assert out[-1].startswith("ERROR session is poisoned")
    s.handle("reset", emit)
    assert out[-1] == "RESET prefix_len=0"
    s.handle("feed " + " ".join(map(str, ids1)), emit)
    s.handle("gen 2", emit)
    assert [int(l.split()[1]) for l in out[-3:-1]] == toks[:2]
    s.handle("frobnicate", emit)
    assert out[-1].startswith("ERROR unknown command 'frobnicate'")
    assert s.handle("quit", emit) is False and out[-1] == "BYE"
    s.close()


def test_session_stdin_stdout():
    cmds = "feed 11 22 33\ngen 3\nstats\nquit\n"
    env = dict(os.environ)
    env["PYTHONPATH"] = f"{ROOT}:{ROOT / 'qwen3.5-0.8b_amd'}"
    r = subprocess.run([sys.executable, "-m", "qwen35.session", "--cap", "256", "--max-rows", "64"],
                       input=cmds, capture_output=True, text=True, timeout=180, env=env)
    assert r.returncode == 0, r.stderr[-2000:]
    # the CLI runs k = 2 rounds by default: drop their diagnostic lines (budget 3 < k + 1 rows
    # skips every round here, so the tokens come from plain steps)
    diag = ("ROUND-SKIP ", "ACCEPT ", "MTPSTAT ")
    lines = [l for l in r.stdout.splitlines() if l and not l.startswith(diag)]
    assert r.stdout.count("ROUND-SKIP reason=budget_tail") == 3
    assert lines[0] == "READY cap=256"
    assert lines[1] == "FED n=3 prefix_len=3"
    assert [l.split()[0] for l in lines[2:6]] == ["GEN", "GEN", "GEN", "END"]
    assert lines[5] == "END steps=3 stop=0 prefix_len=6"
    assert lines[6] == "PREFIX p=6 sampled=-1 stopped=0"
    assert lines[7] == "BYE"


def test_session_mtp_rounds_match_plain(tmp_path, monkeypatch):
    """`gen` by speculative rounds (k = 2) prints the GEN/FED/END lines of the plain session
    over several turns, including accepted drafts and the stop cut. Random weights make the
    drafter disagree always, so the final norms are reshaped to keep one hidden dimension d
    (1 + w = 0 elsewhere) and two embedding rows get large entries in d: every greedy pick
    (target and draft) is then 248046 (the stop token) or 1000 by the sign of x_d. With a
    positive norm factor at d the picks repeat (a fed 1000 adds -8 to x_d): drafts are
    accepted, mostly whole rounds. With a negative factor for the target its picks
    alternate (1000, then the stop token); the drafter's factor takes both signs. A third
    run with the stop cut switched off (stop = -1 passed to the round) must print a
    different transcript for some setting: an accepted stop draft then sits mid-round, so
    the cut was exercised and mattered."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, State
    from qwen35.session import STOP_TOKEN, Session
    d = 7
    keep = ("GEN ", "FED ", "END ")
    feeds = [lane_prompt_ids(11, t, n) for t, n in enumerate((8, 3, 2, 4, 1, 5, 2, 6))]
    eng = Engine(max_rows=64, max_ctx=512, seed=0, use_graph=True)

    def norm_w(factor_bits):
        w = np.full(1024, 0xBF80, np.uint16)          # bf16 -1.0: 1 + w = 0
        w[d] = factor_bits
        return w

    def run(k):
        out = []
        s = Session(eng, 512, str(tmp_path), mtp_k=k)
        for ids in feeds:
            s.handle("feed " + " ".join(str(int(t)) for t in ids), out.append)
            s.handle("gen 24", out.append)
        s.close()
        return out

    try:
        emb = "model.language_model.embed_tokens.weight"
        E = eng.read_tensor(emb, 248320 * 1024).reshape(248320, 1024)
        E[STOP_TOKEN, d] = 0x4100                       # bf16 8.0
        E[1000, d] = 0xC100                             # bf16 -8.0
        eng.load_tensor(emb, E.reshape(-1))
        del E
        cut_mattered, accepted = False, 0
        # (target, drafter) factor 1 + w at d: bf16 bits of w = 3.0 (factor 4) or -5.0 (-4)
        for tgt_bits, mtp_bits in ((0x4040, 0x4040), (0xC0A0, 0x4040), (0xC0A0, 0xC0A0)):
            eng.load_tensor("model.language_model.norm.weight", norm_w(tgt_bits))
            eng.load_tensor("mtp.norm.weight", norm_w(mtp_bits))
            plain_log, spec_log = run(0), run(2)
            orig = State.mtp_round
            monkeypatch.setattr(State, "mtp_round", lambda self, cur, k, lanes=None, stats=None, stop=-1:
                                orig(self, cur, k, lanes, stats, -1))
            nocut = [l for l in run(2) if l.startswith(keep)]
            monkeypatch.undo()
            plain = [l for l in plain_log if l.startswith(keep)]
            spec = [l for l in spec_log if l.startswith(keep)]
            acc = [l for l in spec_log if l.startswith("ACCEPT ")]
            n_acc = [int(l.split("n_accepted=")[1].split()[0]) for l in acc]
            stops = sum(l.startswith("END ") and " stop=1 " in l for l in plain)
            print(f"mtp session (norm bits {tgt_bits:#x}, {mtp_bits:#x}): {len(acc)} rounds, accepted per round "
                  f"{n_acc}, {stops} stopped turns; without the cut the transcript differs: {nocut != plain}",
                  flush=True)
            assert not any(l.startswith("ERROR") for l in plain_log + spec_log)
            assert spec == plain
            assert len(acc) > 0 and any(l.startswith("MTPSTAT ") for l in spec_log)
            cut_mattered |= nocut != plain
            accepted += sum(n_acc)
        assert cut_mattered and accepted > 0
    finally:
        eng.close()


def test_session_adaptive_depth_abandons_and_matches_plain(tmp_path):
    """Random-init weights: the drafter never agrees, so each round emits one token; the
    session's adaptive tracker (engine/mtp_adaptive.h) demotes 2 -> 1 after 16 rounds and abandons
    after 24 more, its estimates billed at this engine's measured round costs (1 / 1.920 and
    1 / 1.552, not the reference's gfx1151 1.90 / 1.58), and the transcript is the plain session's.
    A feed starts a fresh tracker: the next turn speculates at k = 2 again."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine
    from qwen35.session import Session
    keep = ("GEN ", "FED ", "END ")
    eng = Engine(max_rows=64, max_ctx=512, seed=0, use_graph=True)
    try:
        logs = {}
        for k in (0, 2):
            out = []
            s = Session(eng, 512, str(tmp_path), mtp_k=k)
            for t in range(2):
                s.handle("feed " + " ".join(str(x) for x in lane_prompt_ids(21, t, 6)), out.append)
                s.handle("gen 100", out.append)
            s.close()
            logs[k] = out
        assert [l for l in logs[0] if l.startswith(keep)] == [l for l in logs[2] if l.startswith(keep)]
        ad = [l for l in logs[2] if l.startswith("MTPADAPT ")]
        print("adaptive session:", ad, flush=True)
        assert len(ad) == 4                                   # two changes in each of the two turns
        assert "k=1 " in ad[0] and "window_rounds=16 " in ad[0] and "prev_k=2 " in ad[0]
        assert "k=0 " in ad[1] and "window_rounds=24 " in ad[1] and ad[1].endswith("plain=1")
        assert "k=1 " in ad[2] and "k=0 " in ad[3]
        assert f"est={1 / 1.920:.4f} " in ad[0] and f"est={1 / 1.552:.4f} " in ad[1]
        acc = [l for l in logs[2] if l.startswith("ACCEPT ")]
        assert sum(" k=2 " in l for l in acc) == 32 and sum(" k=1 " in l for l in acc) == 48
    finally:
        eng.close()


def test_chat_driver_turns_match_forward(eng, tmp_path):
    """Two text turns through the chat driver (render -> tokenize -> feed -> gen): the reply ids
    equal a plain Forward over the rendered-and-tokenized transcript; the second turn extends
    the first (the im_end close of a budget-ended reply, then the next user turn)."""
    from test_textio import _write_tokenizer
    from qwen35 import Forward, State
    from qwen35.chat import ChatDriver
    from qwen35.session import Session
    from qwen35.textio import Tokenizer
    _write_tokenizer(tmp_path / "tokenizer.json")
    tok = Tokenizer(tmp_path)
    s = Session(eng, 512)
    d = ChatDriver(s, tok)
    p1 = d.prompt_ids("PING")
    g1 = d.turn("PING", max_new=4)
    assert p1[:4] == [248045, 1, 4, 3] and len(g1) == 4 and not d.closed
    p2 = d.prompt_ids("hello")
    assert p2[:2] == [248046, 4]               # the truncated reply is closed first
    g2 = d.turn("hello", max_new=3)
    # the same transcript as one Forward: prompt, the 4 shown replies (each fed; the unshown 5th
    # sample was dropped), then p2
    f = Forward(eng, State(eng, 1, 512))
    ref1 = f.greedy(p1, 3, stop_on_eos=False)
    assert g1 == ref1[:4]
    f2 = Forward(eng, State(eng, 1, 512))
    ref2 = f2.greedy(p1 + g1 + p2, 2, stop_on_eos=False)
    assert g2 == ref2[:3]
    s.close()
