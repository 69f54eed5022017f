"""MTP rounds that accept drafts (mtpaccept::accept_round, engine/mtp_accept.cpp:89; greedy
accept + rollback of speccheck/mtp.py:150-177) at 8 lanes. Random-init drafts never agree
with the target, so the final norms are reshaped to keep one hidden dimension d (1 + w = 0
elsewhere) and two embedding rows get large entries in d: every greedy pick is then token
248046 or 1000 by the sign of x_d, and the drafter agrees with the target often. Two
settings: norm factors +4 / +4 (picks repeat: whole rounds accepted) and -4 / -4 (the
target's picks alternate). Checked per lane against a plain State fed the same tokens one
step at a time: every emitted token is the plain step's argmax, and after the rounds the
GDN state S, the conv window and the K/V rows of both states are bit-identical (the verify
rows and the kept state are those of plain steps: the rollback kept the right pending rows,
window slot and prefix), also after a 70-token prompt wave (the chunked form, which first
applies the lane's pending verify rows to its state)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

D, STOP = 7, 248046


def _norm_w(bits):
    w = np.full(1024, 0xBF80, np.uint16)          # bf16 -1.0: 1 + w = 0
    w[D] = bits
    return w


def test_mtp_rounds_with_accepts_match_plain_steps():
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, State
    eng = Engine(max_rows=64, max_ctx=512, seed=0)
    try:
        emb = "model.language_model.embed_tokens.weight"
        E = eng.read_tensor(emb, 248320 * 1024).reshape(248320, 1024)
        E[STOP, D] = 0x4100                          # bf16 8.0
        E[1000, D] = 0xC100                          # bf16 -8.0
        eng.load_tensor(emb, E.reshape(-1))
        del E
        lanes = 8
        total = np.zeros(4, np.int64)
        hist = {}
        for bits in (0x4040, 0xC0A0):                # w[d] = 3.0 (factor 4), -5.0 (factor -4)
            eng.load_tensor("model.language_model.norm.weight", _norm_w(bits))
            eng.load_tensor("mtp.norm.weight", _norm_w(bits))
            spec = State(eng, lanes, 256, mtp_k=2, mtp_cap=256)
            plain = State(eng, lanes, 256)
            cur = []
            for i in range(lanes):
                ids = lane_prompt_ids(30 + i, 0, 5 + 3 * i)
                y = spec.prefill(i, ids)
                assert plain.prefill(i, ids) == y
                cur.append(int(y))
            for r in range(6):
                stats = np.zeros(4, np.int64)
                print(f"mtp accept: norm bits {bits:#x}, round {r}", flush=True)
                em = spec.mtp_round(cur, 2, list(range(lanes)), stats)
                total += stats
                for i in range(lanes):
                    e = [int(t) for t in em[i]]
                    hist[len(e) - 1] = hist.get(len(e) - 1, 0) + 1
                    fed = [cur[i]] + e[:-1]
                    for j, t in enumerate(fed):
                        got = int(plain.decode_step([t], [i])[0])
                        assert got == e[j], (bits, r, i, j)
                    cur[i] = e[-1]
                    assert spec.prefix_len(i) == plain.prefix_len(i)
            # a prompt wave of >= 64 rows takes the chunked form, which reads a state slot as
            # it stands: lanes with verify rows still pending are brought up to date first
            for i in (0, 3):
                ids = lane_prompt_ids(70 + i, 1, 70)
                assert spec.prefill(i, ids) == plain.prefill(i, ids), (bits, i)
                cur[i] = None
            for i in range(lanes):
                P = plain.prefix_len(i)
                for which in ("S", "win"):
                    assert np.array_equal(spec.read(i, which), plain.read(i, which)), (bits, i, which)
                for which in ("k", "v"):
                    assert np.array_equal(spec.read(i, which, P), plain.read(i, which, P)), (bits, i, which)
            spec.close()
            plain.close()
        print(f"mtp accept: accepted per round histogram {hist}, stats {total.tolist()}", flush=True)
        assert hist.get(2, 0) > 0 and hist.get(0, 0) > 0
    finally:
        eng.close()


def test_adaptive_step_mixed_depths_lossless():
    """q35_mtp_adaptive_step over 24 lanes whose policies start at depths 2, 1 and 0 (all three
    groups in one turn): every lane's emitted stream equals plain greedy steps of the same lane,
    and with random-init weights (no draft accepted) the depths walk 2 -> 1 -> 0 at the policy's
    thresholds (16 rounds at k = 2, 24 at k = 1)."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, MtpPolicy, State
    eng = Engine(max_rows=96, max_ctx=512, seed=0, use_graph=True)
    try:
        n = 24
        spec = State(eng, n, 320, mtp_k=2, mtp_cap=256)
        plain = State(eng, n, 320)
        cur, pref = [], []
        for i in range(n):
            ids = lane_prompt_ids(60 + i, 0, 4 + i % 5)
            y = spec.prefill(i, ids)
            assert plain.prefill(i, ids) == y
            cur.append(int(y))
        pol = [MtpPolicy(2 if i % 3 == 0 else 1 if i % 3 == 1 else 0) for i in range(n)]
        streams = [[c] for c in cur]
        depth_hist = []
        for turn in range(45):
            em, dep = spec.mtp_adaptive_step(cur, pol)
            depth_hist.append(dep.copy())
            for i in range(n):
                streams[i] += [int(t) for t in em[i]]
                cur[i] = int(em[i][-1])
        lens = min(len(s) for s in streams)
        pc = [s[0] for s in streams]
        for step in range(lens - 1):
            pc = [int(t) for t in plain.decode_step(pc)]
            for i in range(n):
                assert pc[i] == streams[i][step + 1], (i, step)
        d = np.array(depth_hist)                  # [turn][lane]
        assert (d[:16, 0] == 2).all() and (d[16:40, 0] == 1).all() and (d[40:, 0] == 0).all()
        assert (d[:24, 1] == 1).all() and (d[24:, 1] == 0).all()
        assert (d[:, 2] == 0).all()
        for p in pol:
            p.close()
        spec.close()
        plain.close()
    finally:
        eng.close()


def test_draft_then_verify_equals_round():
    """The reference's two-call round (mtpdraft::draft_round twice, then mtpaccept::accept_round
    with the candidates) through q35_mtp_draft + q35_mtp_verify gives q35_mtp_round's emits and
    leaves the same state (S, window, K/V, MTP K/V, prefix) bit for bit, over rounds that accept
    no draft and both drafts (the reshaped-norm setting of the test above, factor -4)."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, State
    eng = Engine(max_rows=64, max_ctx=512, seed=0)
    try:
        emb = "model.language_model.embed_tokens.weight"
        E = eng.read_tensor(emb, 248320 * 1024).reshape(248320, 1024)
        E[STOP, D] = 0x4100
        E[1000, D] = 0xC100
        eng.load_tensor(emb, E.reshape(-1))
        del E
        eng.load_tensor("model.language_model.norm.weight", _norm_w(0xC0A0))
        eng.load_tensor("mtp.norm.weight", _norm_w(0xC0A0))
        lanes = 4
        a = State(eng, lanes, 256, mtp_k=2, mtp_cap=256)
        b = State(eng, lanes, 256, mtp_k=2, mtp_cap=256)
        cur = []
        for i in range(lanes):
            ids = lane_prompt_ids(40 + i, 0, 6 + 2 * i)
            y = a.prefill(i, ids)
            assert b.prefill(i, ids) == y
            cur.append(int(y))
        ca, cb, seen = list(cur), list(cur), set()
        for r in range(6):
            print(f"draft + verify: round {r}", flush=True)
            ea = a.mtp_round(ca, 2)
            P = [b.prefix_len(i) for i in range(lanes)]
            d1, _, _ = b.mtp_draft(cb, [p + 1 for p in P], 0)
            d2, _, _ = b.mtp_draft(d1, [p + 2 for p in P], 1)
            eb = b.mtp_verify(cb, np.stack([d1, d2], 1))
            assert [list(map(int, x)) for x in ea] == [list(map(int, x)) for x in eb], r
            seen |= {len(x) - 1 for x in ea}
            ca = [int(x[-1]) for x in ea]
            cb = [int(x[-1]) for x in eb]
        for i in range(lanes):
            n = a.prefix_len(i)
            assert n == b.prefix_len(i)
            for w in ("S", "win"):
                assert np.array_equal(a.read(i, w), b.read(i, w)), (i, w)
            for w in ("k", "v"):
                assert np.array_equal(a.read(i, w, n), b.read(i, w, n)), (i, w)
            for w in ("mk", "mv"):
                assert np.array_equal(a.read(i, w, 8), b.read(i, w, 8)), (i, w)
        print("accepted drafts per round seen:", sorted(seen), flush=True)
        assert {0, 2} <= seen
        a.close()
        b.close()
    finally:
        eng.close()
