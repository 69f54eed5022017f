"""Resident session line protocol over the MI355X engine (one lane, weights and state stay on
the GPU across turns): the protocol of the reference's `decode_run --session`
(engine/decode_run.cpp:1760-1790 spec, 2390-2680 loop) that engine/chat.py drives.

    python -m qwen35.session [--cap 4096] [--checkpoint DIR | --seed 0] [--out DIR]

prints `READY cap=<n>`, then answers one command per stdin line:

    feed <id> ...      one prompt pass over [pending sample] + ids -> "FED n=<k> prefix_len=<P>"
    gen <n>            up to n greedy tokens, each streamed as "GEN <id> <pos>", then
                       "END steps=<k> stop=<0|1> prefix_len=<P>"; token 248046 ends the turn
    reset              fresh request -> "RESET prefix_len=0"
    stats              "PREFIX p=<P> sampled=<id> stopped=<0|1>"
    dump <pos> | dump <min> <max> | dump off
                       opt-in f32 logits rows (one file per priced row whose position is in the
                       window, written to --out) with a "DUMP seq= kind= pos= emitted= ..." line
    quit | bye         "BYE"

Token ids only: rendering and tokenizing the chat is the caller's side (engine/chat.py). A
failure inside a step poisons the session until `reset` (the state may be half-advanced);
argument errors do not.

With `--mtp-k K` (K >= 1; the reference's session runs accept rounds at k = 2 by default,
engine/decode_run.cpp:162-187) `gen` advances by speculative rounds instead of single steps,
as mtpaccept::session_body does (engine/mtp_accept.cpp:530-660): a round feeds the pending
sample plus K drafts and prints the accepted drafts, the bonus becoming the next pending
sample; it runs only when the turn can print all K + 1 of its tokens and the lane has room
for K + 1 more slots, else the step is a plain one ("ROUND-SKIP reason=budget_tail" /
"context_limit"); an accepted stop token ends the round's emits and stays pending (the stop
cut). Greedy rounds are lossless, so the GEN lines are those of the plain session; each
round adds an "ACCEPT ..." line and a turn that ran rounds ends with "MTPSTAT ...". While a
logits dump is armed, steps are plain (one priced row per printed token). The drafter's own
K/V cache is kept across feeds (the reference clears it at a feed); that changes which
drafts are proposed, never the tokens printed.

The depth of each round is adaptive by default, as the reference's session runs it
(`--mtp-adaptive 1`, engine/decode_run.cpp:189-198, engine/mtp_adaptive.h): --mtp-k is the
ceiling, the request's tracker demotes 2 -> 1 -> plain steps from what its rounds emitted
("MTPADAPT round= k= est= prev_k= window_rounds= plain=" on each change), and a `feed` or
`reset` starts a fresh tracker (engine/decode_run.cpp:2478-2483, 2510-2516).
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np

from .engine import MI355X_ROUND_COST, VOCAB, Engine, EngineError, MtpPolicy, State

STOP_TOKEN = 248046                  # engine/decode_step.h:492 (kStopToken)
DEFAULT_CAP = 4096                   # engine/decode_run.cpp:72 (kSessionDefaultCap)


class Session:
    """One lane's session state machine; `handle` runs one command line and passes every
    output line to `emit` as soon as it exists (GEN lines stream)."""

    def __init__(self, eng: Engine, cap: int = DEFAULT_CAP, out_dir: str | None = None, mtp_k: int = 0,
                 adaptive: bool = True):
        self.eng = eng
        self.cap = cap
        self.mtp_k = mtp_k
        self.adaptive = adaptive and mtp_k > 0
        self.policy = self._policy() if self.adaptive else None
        self.state = State(eng, 1, cap, mtp_k=mtp_k, mtp_cap=cap if mtp_k else 0)
        self.rounds = 0
        self.turn = np.zeros(4, np.int64)     # drafted, accepted, bonus, verified rows this turn
        self.sampled = -1            # the last sample handed to the caller and not yet consumed
        self.stopped = False
        self.poisoned = False
        self.out_dir = out_dir
        self.lo, self.hi, self.seq = 0, -1, 0

    def _new_turn(self):
        """A fresh adaptive tracker (mtpaccept::session_new_turn, engine/mtp_accept.cpp:501-504)."""
        if self.adaptive:
            self.policy.close()
            self.policy = self._policy()

    def _policy(self) -> MtpPolicy:
        """A fresh tracker billing rounds at this engine's measured round costs."""
        return MtpPolicy(self.mtp_k, MI355X_ROUND_COST[1], MI355X_ROUND_COST[2])

    def ready_line(self) -> str:
        return f"READY cap={self.cap}"

    def close(self):
        self.state.close()
        if self.policy is not None:
            self.policy.close()

    # ---------------------------------------------------------------- logits dump
    def _armed(self) -> bool:
        return bool(self.out_dir) and self.hi >= self.lo

    def _dump(self, emit, kind: str, row: np.ndarray | None, pos: int):
        if not self._armed() or not (self.lo <= pos <= self.hi):
            return
        if row is None:
            emit(f"DUMP-MISS kind={kind} pos0={pos} rows=1 reason=no-logits")
            return
        self.seq += 1
        name = f"session_{self.seq:06d}_{kind}_{pos}.bin"
        np.ascontiguousarray(row, dtype=np.float32).tofile(Path(self.out_dir) / name)
        emit(f"DUMP seq={self.seq} kind={kind} pos={pos} emitted=1 vocab={VOCAB} bytes={VOCAB * 4} file={name}")

    # ---------------------------------------------------------------- commands
    def handle(self, line: str, emit) -> bool:
        """Runs one command; returns False after quit/bye."""
        words = line.split()
        if not words:
            return True
        cmd, args = words[0], words[1:]
        if cmd in ("quit", "bye"):
            emit("BYE")
            return False
        if cmd == "reset":
            self.state.reset([0])
            self._new_turn()
            self.sampled, self.stopped, self.poisoned = -1, False, False
            emit("RESET prefix_len=0")
            return True
        if self.poisoned:
            emit("ERROR session is poisoned by the failed step: send reset before the next feed or gen")
            return True
        # argument errors are the caller's and do not poison the session
        if cmd == "gen" and self.sampled < 0:
            emit("ERROR gen with no sampled token: feed this turn's prompt first")
            return True
        budget = 0
        if cmd == "gen":
            try:
                budget = int(args[0])
            except (IndexError, ValueError):
                emit("ERROR gen needs a token count")
                return True
        try:
            if cmd == "feed":
                self._new_turn()
                toks = [self.sampled] if self.sampled >= 0 else []
                for w in args:               # ids up to the first word that is not one
                    try:
                        toks.append(int(w))
                    except ValueError:
                        break
                want = self._armed()
                y = self.state.prefill(0, toks, logits=want)
                y0, row = (y if want else (y, None))
                p = self.state.prefix_len(0)
                emit(f"FED n={len(toks)} prefix_len={p}")
                self.sampled = int(y0)
                self._dump(emit, "feed", row, p - 1)
            elif cmd == "gen":
                emitted, stop, cur = 0, False, self.sampled
                self.turn[:] = 0
                while emitted < budget:
                    emit(f"GEN {cur} {self.state.prefix_len(0) - 1}")
                    emitted += 1
                    if cur == STOP_TOKEN:
                        stop = True
                        break
                    want = self._armed()
                    k = self.policy.k if self.adaptive else self.mtp_k
                    if k and not want:
                        p = self.state.prefix_len(0)
                        rows = k + 1
                        if p + rows > self.cap:
                            emit(f"ROUND-SKIP reason=context_limit anchor={p} cap={self.cap} rows={rows}")
                        elif budget - emitted < rows:
                            emit(f"ROUND-SKIP reason=budget_tail anchor={p} budget_left={budget - emitted} rows={rows}")
                        else:
                            em = [int(t) for t in self.state.mtp_round([cur], k, [0], self.turn, STOP_TOKEN)[0]]
                            self.rounds += 1
                            a = len(em) - 1
                            emit(f"ACCEPT round={self.rounds} anchor={p} fed={cur} k={k} n_accepted={a} "
                                 f"emitted={len(em)} pos={p}->{self.state.prefix_len(0)}")
                            if self.adaptive:
                                ch, est = self.policy.note(k, len(em))
                                if ch:
                                    emit(f"MTPADAPT round={self.rounds} k={ch[1]} est={est:.4f} prev_k={ch[0]} "
                                         f"window_rounds={ch[2]} plain={int(ch[1] == 0)}")
                            for i, t in enumerate(em[:-1]):    # the accepted drafts (fed, so shown now)
                                emit(f"GEN {t} {p + i}")
                                emitted += 1
                            cur = em[-1]
                            continue
                    
                    out = self.state.decode_step([cur], logits=want)
                    tok, lg = (out if want else (out, None))
                    cur = int(tok[0])
                    self._dump(emit, "step", None if lg is None else lg[0], self.state.prefix_len(0) - 1)
                # stop: the stop token stays pending (the next feed consumes it); budget: the last
                # sample was never shown, so it is dropped and the caller closes the turn
                self.sampled = cur if stop else -1
                self.stopped = stop
                if self.turn[2]:
                    d, acc, rounds = int(self.turn[0]), int(self.turn[1]), int(self.turn[2])
                    emit(f"MTPSTAT rounds={rounds} drafted={d} accepted={acc} "
                         f"accept_rate={acc / d:.4f} tokens_per_round={(acc + rounds) / rounds:.4f}")
                emit(f"END steps={emitted} stop={int(stop)} prefix_len={self.state.prefix_len(0)}")
            elif cmd == "stats":
                emit(f"PREFIX p={self.state.prefix_len(0)} sampled={self.sampled} stopped={int(self.stopped)}")
            elif cmd == "dump":
                if not args:
                    emit("ERROR dump needs `dump <pos>`, `dump <min> <max>` or `dump off`")
                elif args[0] == "off":
                    self.hi = self.lo - 1
                    emit(f"DUMP armed=0 written={self.seq}")
                elif not self.out_dir:
                    emit("ERROR dump needs --out DIR: the rows go beside the other dumps")
                else:
                    try:
                        a = int(args[0])
                    except ValueError:
                        emit(f"ERROR dump position must be an integer, got '{args[0]}'")
                        return True
                    try:
                        b = int(args[1]) if len(args) > 1 else a
                    except ValueError:
                        b = a
                    if b < a:
                        emit(f"ERROR dump window is empty: max={b} is below min={a}")
                    else:
                        self.lo, self.hi = a, b
                        emit(f"DUMP armed=1 min={a} max={b} dir={self.out_dir}")
            else:
                emit(f"ERROR unknown command '{cmd}' (feed|gen|reset|stats|dump|quit)")
        except EngineError as e:
            self.poisoned = True
            emit(f"ERROR {e}")
        return True


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="resident session line protocol (decode_run --session)")
    ap.add_argument("--cap", type=int, default=DEFAULT_CAP, help="cache slots of the session's lane")
    ap.add_argument("--checkpoint", help="directory holding the model's .safetensors file")
    ap.add_argument("--seed", type=int, default=0, help="seeded random-init weights when no checkpoint is given")
    ap.add_argument("--max-rows", type=int, default=512, help="rows per prompt wave")
    ap.add_argument("--out", help="directory for opt-in logits dumps")
    ap.add_argument("--graph", type=int, default=1, help="capture decode steps in hipGraphs")
    ap.add_argument("--mtp-k", type=int, default=2, help="drafts per speculative round; 0: plain steps")
    ap.add_argument("--mtp-adaptive", type=int, default=1, choices=(0, 1),
                    help="1: each round's depth from the request's own accept history (engine/mtp_adaptive.h)")
    a = ap.parse_args(argv)
    eng = Engine(max_rows=a.max_rows, max_ctx=a.cap, seed=None if a.checkpoint else a.seed, use_graph=bool(a.graph))
    if a.checkpoint:
        n, sk = eng.load_checkpoint(a.checkpoint)
        print(f"LOADED tensors={n} skipped={sk}", flush=True)
    s = Session(eng, a.cap, a.out, mtp_k=a.mtp_k, adaptive=bool(a.mtp_adaptive))

    def emit(line: str):
        print(line, flush=True)

    emit(s.ready_line())
    try:
        for line in sys.stdin:
            if not s.handle(line, emit):
                break
    finally:
        s.close()
        eng.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
