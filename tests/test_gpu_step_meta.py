"""Decode-step metadata left on the device: a decode step advances its rows' positions,
slots and state-slot indices on the device and leaves its sampled tokens in the token row,
so the next step of the same state and lanes, fed exactly those tokens, skips the metadata
upload. Checked against steps that always upload (the same sequence with a step of another
state in between, which invalidates the device copy): same tokens and bit-identical logits,
across greedy runs, a fed token other than the sampled one (teacher forcing), a change of
the lane set, a reset lane, a prefill, an MTP round, a lane copy and a snapshot restore in
between, with captured (graph) and eager steps."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("graph", [True, False])
def test_device_metadata_fast_path_matches_uploads(graph):
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, State
    eng = Engine(max_rows=64, max_ctx=512, seed=0, use_graph=graph)
    try:
        a = State(eng, 4, 256, mtp_k=2, mtp_cap=128)   # consecutive steps: device metadata reused
        b = State(eng, 4, 256, mtp_k=2, mtp_cap=128)   # same work, another state's step in between
        other = State(eng, 1, 64)
        other.prefill(0, [5, 6, 7])
        o_tok = [9]
        prompts = [lane_prompt_ids(40 + i, 0, 6 + i) for i in range(4)]
        for st in (a, b):
            for i in range(4):
                st.prefill(i, prompts[i])
        script = []                            # (tokens or None = feed back, lanes)
        script += [(None, [0, 1, 2, 3])] * 5
        script += [([11, 12, 13, 14], [0, 1, 2, 3])]           # teacher forcing
        script += [(None, [0, 1, 2, 3])] * 3
        script += [(None, [1, 3])] * 3                          # lane subset
        script += [("reset2", None)]
        script += [(None, [0, 1, 3])] * 3
        script += [("prefill", None)]
        script += [(None, [0, 1, 2, 3])] * 4
        script += [("snap1", None)]
        script += [("mtp01", None)]
        script += [(None, [0, 1, 2, 3])] * 3
        script += [("copy0to3", None)]
        script += [(None, [0, 1, 2, 3])] * 3
        script += [("restore1", None)]
        script += [(None, [0, 1, 2, 3])] * 3
        last = {}
        for st, interleave in ((a, False), (b, True)):
            out = []
            prev = {i: None for i in range(4)}
            snap = None
            for k, (toks, lanes) in enumerate(script):
                print(f"step meta: graph={graph} {'upload' if interleave else 'device'} step {k} {toks}", flush=True)
                if toks == "snap1":
                    snap = (st.snapshot(1), prev[1])
                    continue
                if toks == "restore1":
                    st.restore(1, snap[0])
                    prev[1] = snap[1]
                    continue
                if toks == "copy0to3":
                    st.copy_lane(0, st, 3)
                    prev[3] = prev[0]
                    continue
                if toks == "mtp01":
                    em = st.mtp_round([prev[0], prev[1]], 2, [0, 1])
                    prev[0], prev[1] = int(em[0][-1]), int(em[1][-1])
                    out.append((em, None))
                    continue
                if toks == "reset2":
                    st.reset([2])
                    continue
                if toks == "prefill":
                    st.prefill(2, lane_prompt_ids(50, 0, 4))
                    prev[2] = None
                    continue
                if toks is None:
                    toks = [prev[l] if prev[l] is not None else 100 + l for l in lanes]
                if interleave:
                    o_tok = list(other.decode_step(o_tok, [0]))
                t, lg = st.decode_step(toks, lanes, logits=True)
                for l, x in zip(lanes, t):
                    prev[l] = int(x)
                out.append((list(map(int, t)), lg))
            last[interleave] = out
        for (ta, la), (tb, lb) in zip(last[False], last[True]):
            assert ta == tb
            assert (la is None and lb is None) or np.array_equal(la, lb)
        for st in (a, b, other):
            st.close()
    finally:
        eng.close()
