"""Prefix reuse and preempt / resume (specification/08-state-management.md §08.3-08.4: the
per-request tuple is stored and restored verbatim, no recompute): a lane forked device to
device (q35_state_copy_lane) or restored from a host snapshot continues exactly as a lane that
ran the whole transcript itself -- tokens, logits and state bit for bit, MTP rounds included --
and refused copies (capacity, corrupt blob) raise."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    from qwen35 import Engine
    e = Engine(max_rows=64, max_ctx=512, seed=0, use_graph=True)
    yield e
    e.close()


def _run(st, lane, ids_more, steps):
    """prefill ids_more into `lane`, then `steps` decodes of that lane; tokens + logits."""
    y, lg = st.prefill(lane, ids_more, logits=True)
    out, lgs = [y], [lg]
    for _ in range(steps):
        t, l = st.decode_step([out[-1]], lanes=[lane], logits=True)
        out.append(int(t[0]))
        lgs.append(l[0])
    return out, lgs


def test_prefix_fork_and_snapshot(eng):
    from oracle.weights import lane_prompt_ids
    from qwen35 import EngineError, State
    ids = [int(t) for t in lane_prompt_ids(21, 0, 30)]
    ref = State(eng, 1, 256)
    rt, rl = _run(ref, 0, ids, 3)
    cache = State(eng, 1, 256)
    cache.prefill(0, ids[:20])                       # the shared prefix
    b = State(eng, 4, 300)
    cache.copy_lane(0, b, 2)
    assert b.prefix_len(2) == 20 and b.prefix_len(0) == 0
    bt, bl = _run(b, 2, ids[20:], 3)
    assert bt == rt and all(np.array_equal(x, y) for x, y in zip(bl, rl))
    assert np.array_equal(b.read(2, "S"), ref.read(0, "S"))
    assert np.array_equal(b.read(2, "k", 33), ref.read(0, "k", 33))
    assert np.array_equal(b.read(2, "v", 33), ref.read(0, "v", 33))

    blob = b.snapshot(2)                             # preempt lane 2, resume elsewhere
    d = State(eng, 2, 256)
    d.restore(1, blob)
    assert d.prefix_len(1) == 33
    t1, l1 = [], []
    for st, ln in ((b, 2), (d, 1)):
        cur = bt[-1]
        toks, lgs = [], []
        for _ in range(3):
            t, l = st.decode_step([cur], lanes=[ln], logits=True)
            cur = int(t[0])
            toks.append(cur)
            lgs.append(l[0])
        t1.append(toks)
        l1.append(lgs)
    assert t1[0] == t1[1] and all(np.array_equal(x, y) for x, y in zip(l1[0], l1[1]))
    assert np.array_equal(b.read(2, "S"), d.read(1, "S"))

    small = State(eng, 1, 16)
    with pytest.raises(EngineError, match="capacity"):
        b.copy_lane(2, small, 0)
    bad = blob.copy()
    bad[:8] = 0
    with pytest.raises(EngineError, match="snapshot"):
        d.restore(0, bad)
    with pytest.raises(EngineError):
        d.restore(0, blob[:-100])
    for s in (ref, cache, b, d, small):
        s.close()


def test_fork_with_mtp_cache(eng):
    from oracle.weights import lane_prompt_ids
    from qwen35 import State
    ids = [int(t) for t in lane_prompt_ids(22, 0, 16)]
    a = State(eng, 1, 256, mtp_k=2, mtp_cap=64)
    cur = a.prefill(0, ids)
    em = a.mtp_round([cur], 2)
    cur = em[0][-1]
    b = State(eng, 3, 256, mtp_k=2, mtp_cap=64)
    a.copy_lane(0, b, 1)
    snap = a.snapshot(0)
    c = State(eng, 1, 256, mtp_k=2, mtp_cap=64)
    c.restore(0, snap)
    outs = []
    for st, ln in ((a, 0), (b, 1), (c, 0)):
        t, seq = cur, []
        for _ in range(3):
            e = st.mtp_round([t], 2, lanes=[ln])[0]
            seq.append(list(e))
            t = e[-1]
        outs.append((seq, st.read(ln, "S"), st.read(ln, "mk", 2)))   # the last drafts' slots
    for o in outs[1:]:
        assert o[0] == outs[0][0]
        assert np.array_equal(o[1], outs[0][1]) and np.array_equal(o[2], outs[0][2])
    for s in (a, b, c):
        s.close()


@pytest.mark.parametrize("exact", [0, 1])
def test_prefill_lanes_equals_one_lane_prefills(exact):
    """q35_prefill_lanes (prompts of several lanes sharing body passes, ragged lengths, more
    rows than max_rows so rounds split) against q35_prefill of each lane alone: greedy ids and
    logits rows equal, and every lane's state (S, window, K/V, prefix) bit-identical. Prompts
    under 64 tokens take the same kernels both ways; with prompt_exact the long prompt's waves
    do too, so then the long lane is bit-identical as well (else within the engine tolerance)."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, State
    e = Engine(max_rows=64, max_ctx=512, seed=0)
    try:
        e.set_option("prompt_exact", exact)
        lens = [5, 17, 1, 40, 9, 90]
        prompts = [lane_prompt_ids(60 + i, 0, L) for i, L in enumerate(lens)]
        lanes = [3, 0, 5, 1, 4, 2]
        a = State(e, 6, 256)
        y, lg = a.prefill_lanes(prompts, lanes, logits=True)
        b = State(e, 6, 256)
        for i, (p, ln) in enumerate(zip(prompts, lanes)):
            yb, lb = b.prefill(ln, p, logits=True)
            same = exact or len(p) < 64
            if same:
                assert int(y[i]) == int(yb) and np.array_equal(lg[i], lb), i
            else:
                assert np.abs(lg[i] - lb).max() <= 0.375, i
            assert a.prefix_len(ln) == b.prefix_len(ln) == len(p)
            if same:
                for w in ("S", "win"):
                    assert np.array_equal(a.read(ln, w), b.read(ln, w)), (i, w)
                for w in ("k", "v"):
                    assert np.array_equal(a.read(ln, w, len(p)), b.read(ln, w, len(p))), (i, w)
        # and the lanes decode on from there as the one-lane states do
        t = a.decode_step([int(v) for v in y], lanes)
        tb = b.decode_step([int(v) for v in y], lanes)
        short = [i for i, p in enumerate(prompts) if exact or len(p) < 64]
        assert all(int(t[i]) == int(tb[i]) for i in short)
        a.close()
        b.close()
    finally:
        e.close()
