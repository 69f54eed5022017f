"""Deferred GDN state writes (engine option gdn_defer): a decode step keeps a lane's state update
as a pending factor row for up to gdn_defer steps and writes the state on the next one; the rows
are replayed with the recurrence's own rounded operations, so a deferring engine must give the
bits of one that writes the state every step. Checked at 64 lanes (the persistent GDN kernel)
and at 1 lane (the column-sliced kernel): tokens and logits of every step, the GDN state read in
the middle of a cycle (pending rows applied by the materialize kernel) and at its end, an MTP
verify round on top of pending decode rows, a lane copy and a snapshot with rows pending."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lanes", [64, 1])
def test_deferred_gdn_writes_bit_identical(lanes):
    from qwen35 import Engine, State
    L = 200
    engs, sts = [], []
    for d in (0, 3):
        eng = Engine(max_rows=3 * max(lanes, 64), max_ctx=512, seed=0, use_graph=True)
        eng.set_option("gdn_defer", d)
        st = State(eng, lanes, 320, mtp_k=2, mtp_cap=64)
        st.seed(7, L)
        engs.append(eng)
        sts.append(st)
    rng = np.random.default_rng(3)
    tok = [rng.integers(0, 248320, size=lanes).astype(np.int32)] * 2
    probe = [0, lanes - 1] if lanes > 1 else [0]
    for step in range(11):
        print(f"gdn defer: lanes={lanes} step {step}", flush=True)
        outs = [st.decode_step(t, logits=True) for st, t in zip(sts, tok)]
        assert np.array_equal(outs[0][0], outs[1][0]), f"tokens differ at step {step}"
        assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32)), f"logits differ at step {step}"
        tok = [np.asarray(o[0], np.int32) for o in outs]
        if step in (1, 5, 7):      # mid-cycle (rows pending) and at a cycle's end
            for ln in probe:
                s0, s1 = sts[0].read(ln, "S"), sts[1].read(ln, "S")
                assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32)), f"S of lane {ln} at step {step}"
                w0, w1 = sts[0].read(ln, "win"), sts[1].read(ln, "win")
                assert np.array_equal(w0.view(np.uint32), w1.view(np.uint32)), f"window of lane {ln} at step {step}"
    # pending decode rows under an MTP verify round, then more steps
    for st in sts:
        st.decode_step(np.full(lanes, 17, np.int32))
    ems = [st.mtp_round([int(x) for x in t], 2) for st, t in zip(sts, tok)]
    assert [list(e) for e in ems[0]] == [list(e) for e in ems[1]]
    tok = [np.array([e[-1] for e in em], np.int32) for em in ems]
    for step in range(3):
        outs = [st.decode_step(t, logits=True) for st, t in zip(sts, tok)]
        assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32)), f"logits after MTP, step {step}"
        tok = [np.asarray(o[0], np.int32) for o in outs]
    # rows pending in the source of a copy and of a snapshot
    for st in sts:
        st.decode_step(np.full(lanes, 23, np.int32))
    if lanes > 1:
        for st in sts:
            st.copy_lane(0, st, lanes - 1)
    blobs = [st.snapshot(0) for st in sts]
    assert np.array_equal(blobs[0], blobs[1])
    outs = [st.decode_step(np.full(lanes, 29, np.int32), logits=True) for st in sts]
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))
    for ln in probe:
        assert np.array_equal(sts[0].read(ln, "S").view(np.uint32), sts[1].read(ln, "S").view(np.uint32))
    for st, eng in zip(sts, engs):
        st.close()
        eng.close()
