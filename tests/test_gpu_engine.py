"""End-to-end parity of the engine against the torch-CPU oracle (a restatement of the
reference's speccheck/specimpl.py, itself pinned bit-exact to vectors written from the
reference in tests/golden/).

Tolerances (bf16 path, stated here and checked). They are set at ~1.5x the spread of
the reference's own torch-CPU path between two x86 hosts (this container vs the GPU box,
same weights and ids): logits max |d| 0.22, mean |d| 0.034 over config 0.
  * logits: max |engine - oracle| <= 0.375 and mean |diff| <= 0.05 on teacher-forced steps
    (logits are ~N(0,1.3) bf16 values; 1 bf16 ulp at 4..8 is 0.03125)
  * greedy ids: identical wherever the oracle's top-1/top-2 gap exceeds 0.375
  * GDN fp32 state after the prompt: max |diff| <= 2e-2, relative Frobenius error <= 6e-2
    (the layer inputs themselves differ at bf16 level by then, so this grows with depth)
Bit-exact by construction (checked exactly): batched lane == single lane, prompt-then-
decode == longer prompt (incremental == batch), MTP greedy == plain greedy."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_MAX, LOGIT_MEAN, GAP = 0.375, 0.05, 0.375
# against the reference's own rows (built in the same container as the golden vectors) the
# spread is smaller than against the GPU host's oracle run: measured top-32 max |d| 0.1875
GOLDEN_MAX = 0.25


@pytest.fixture(scope="module")
def eng():
    import torch
    assert torch.cuda.is_available()
    from qwen35 import Engine
    e = Engine(max_rows=128, max_ctx=512, seed=0)
    yield e
    e.close()


@pytest.fixture(scope="module")
def oracle_run(oracle_weights, golden):
    from oracle import model
    ids = [int(t) for t in golden["config0_greedy"]["prompt"]]
    f = model.Forward(oracle_weights)
    rows = []
    toks = f.greedy(ids, 64, stop_on_eos=False, logits_out=rows)
    # torch's CPU bf16 GEMM takes a CPU-dependent path (e.g. AVX512-BF16), so the oracle
    # is pinned to the golden vectors in the CPU suite of the build container, and here it
    # is this host's own instance of the same algorithm.
    gold = [int(t) for t in golden["config0_greedy"]["tokens"]]
    same = next((i for i, (a, b) in enumerate(zip(toks, gold)) if a != b), len(gold))
    print(f"oracle on this host: {same}/65 ids equal to the golden run", flush=True)
    return ids, toks, [r.float().numpy() for r in rows], f


def test_weights_match_oracle(eng, oracle_weights):
    from oracle.weights import registry
    import torch
    for name, shape, kind in registry():
        n = int(np.prod(shape))
        if n > 5_000_000:
            continue
        got = eng.read_tensor(name, n)
        want = oracle_weights.p[name].contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)
        assert np.array_equal(got, want), name
    e = eng.read_tensor("model.language_model.embed_tokens.weight", 248320 * 1024)
    want = oracle_weights.p["model.language_model.embed_tokens.weight"].view(torch.int16).numpy().view(np.uint16).reshape(-1)
    assert np.array_equal(e, want)


def test_teacher_forced_logits(eng, oracle_run):
    from qwen35 import State, Forward
    ids, toks, rows, _ = oracle_run
    st = State(eng, 1, 512)
    f = Forward(eng, st)
    y0, lg = f.prefill(ids, logits=True)
    errs = [np.abs(lg - rows[0])]
    mism = []
    for s in range(64):
        t, lg = f.decode(toks[s], logits=True)
        errs.append(np.abs(lg - rows[s + 1]))
        ref = rows[s + 1]
        top2 = np.sort(ref)[-2:]
        if top2[1] - top2[0] > GAP and t != toks[s + 1]:
            mism.append(s)
        # argmax is bit-exact given the engine's logits
        assert t == int(np.flatnonzero(lg == lg.max())[0])
    mx = max(e.max() for e in errs)
    mean = float(np.mean([e.mean() for e in errs]))
    print(f"teacher-forced logits: max|d|={mx:.4f} mean|d|={mean:.5f}", flush=True)
    assert mx <= LOGIT_MAX and mean <= LOGIT_MEAN
    assert not mism, mism


def test_teacher_forced_vs_reference_golden(eng, golden):
    """The engine against the reference's own bits (tests/golden/config0_greedy.npz, written by
    speccheck/specimpl.py:496-517 in the build container): the prompt, then the reference's 64
    greedy tokens fed back (teacher forcing), so every one of the 65 logits rows is the row the
    reference priced.
      * logits at the reference's top-32 ids of every row within GOLDEN_MAX of its values, mean
        |d| over all rows within LOGIT_MEAN; logits0 / logits64 (the first 4,096 vocabulary
        entries of rows 0 and 64) the same
      * argmax == the reference's token on every row whose reference top-1/top-2 gap exceeds
        GAP, and on every row whose gap exceeds twice that row's measured max |d| over the
        top-32 ids (no plausible rounding difference could reorder such a row); rows that
        pass neither are named as near-ties"""
    from qwen35 import State, Forward
    g = golden["config0_greedy"]
    ids = [int(t) for t in g["prompt"]]
    gold = [int(t) for t in g["tokens"]]
    top_i, top_v = g["top_i"], g["top_v"]
    st = State(eng, 1, 512)
    f = Forward(eng, st)
    y0, lg = f.prefill(ids, logits=True)
    rows, toks = [lg], [y0]
    for s in range(64):
        t, lg = f.decode(gold[s], logits=True)
        rows.append(lg)
        toks.append(t)
    st.close()
    maxes, means, skipped, bad = [], [], [], []
    for r in range(65):
        d = np.abs(rows[r][top_i[r]] - top_v[r])
        maxes.append(float(d.max()))
        means.append(float(d.mean()))
        gap = float(top_v[r][0] - top_v[r][1])
        assert toks[r] == int(np.flatnonzero(rows[r] == rows[r].max())[0])   # lowest id of the max
        if gap > GAP or gap > 2 * d.max():
            if toks[r] != gold[r]:
                bad.append((r, toks[r], gold[r], gap, float(d.max())))
        else:
            skipped.append((r, round(gap, 4), round(float(d.max()), 4)))
        print(f"row {r:2d}: max|d|={d.max():.4f} mean|d|={d.mean():.5f} gap={gap:.4f} "
              f"{'ok' if toks[r] == gold[r] else 'differs'}", flush=True)
    d0 = np.abs(rows[0][:4096] - g["logits0"])
    d64 = np.abs(rows[64][:4096] - g["logits64"])
    print(f"top-32 over 65 rows: max|d|={max(maxes):.4f} mean|d|={np.mean(means):.5f}; "
          f"logits0 max {d0.max():.4f} mean {d0.mean():.5f}; logits64 max {d64.max():.4f} "
          f"mean {d64.mean():.5f}; near-ties not checked (row, gap, max|d|): {skipped}", flush=True)
    assert not bad, bad
    assert max(maxes) <= GOLDEN_MAX and np.mean(means) <= LOGIT_MEAN
    for d in (d0, d64):
        assert d.max() <= GOLDEN_MAX and d.mean() <= LOGIT_MEAN


def _golden_near_tie(golden, r):
    """Row r of the reference's config-0 run is a near-tie: its top-1/top-2 gap is at most GAP
    (two correct bf16 implementations may order it differently)."""
    tv = golden["config0_greedy"]["top_v"][r]
    return float(tv[0] - tv[1]) <= GAP


def test_free_running_greedy(eng, oracle_run, golden):
    """Free-running greedy ids equal the reference's 65 golden ids up to the first divergence,
    and that divergence (if any) is at a row that the reference itself prices as a near-tie;
    the same rule against this host's oracle run."""
    from qwen35 import State, Forward
    ids, toks, rows, _ = oracle_run
    gold = [int(t) for t in golden["config0_greedy"]["tokens"]]
    st = State(eng, 1, 512)
    got = Forward(eng, st).greedy(ids, 64, stop_on_eos=False)
    st.close()
    agree = next((i for i, (a, b) in enumerate(zip(got, gold)) if a != b), 65)
    print(f"free-running greedy: {agree}/65 identical to the reference's golden ids", flush=True)
    if agree < 65:
        assert _golden_near_tie(golden, agree), (agree, golden["config0_greedy"]["top_v"][agree][:2])
    agree_h = next((i for i, (a, b) in enumerate(zip(got, toks)) if a != b), 65)
    print(f"free-running greedy: {agree_h}/65 identical to this host's oracle run", flush=True)
    if agree_h < 65:
        top2 = np.sort(rows[agree_h])[-2:]
        assert top2[1] - top2[0] <= GAP, (agree_h, top2)


def test_gdn_state_after_prompt(eng, oracle_weights, golden):
    import torch
    from oracle import model
    from qwen35 import State
    ids = [int(t) for t in golden["config0_greedy"]["prompt"]][:16]
    f = model.Forward(oracle_weights)
    f.prefill(ids)
    st = State(eng, 1, 512)
    st.prefill(0, ids)
    S = st.read(0, "S")
    for gi, l in enumerate([l for l in range(24) if l % 4 != 3]):
        ref = f.rec[l].numpy()
        d = np.abs(S[gi] - ref)
        rel = np.linalg.norm(S[gi] - ref) / np.linalg.norm(ref)
        assert d.max() <= 2e-2 and rel <= 6e-2, (l, d.max(), rel)
    w = st.read(0, "win")
    for gi, l in enumerate([l for l in range(24) if l % 4 != 3]):
        ref = f.conv_win[l].float().numpy()      # raw projections: bf16 GEMM outputs
        if gi == 0:
            assert np.all(np.abs(w[gi] - ref) <= np.abs(ref) * 2 ** -7 + 2e-3), l
        else:                                    # deeper layers see already-diverged inputs
            assert np.abs(w[gi] - ref).mean() <= 0.05 * np.abs(ref).mean(), l
    k = st.read(0, "k", len(ids))
    kf = (k.astype(np.uint32) << 16).view(np.float32)
    for ai, l in enumerate([3, 7, 11, 15, 19, 23]):
        ref = torch.cat(f.kv[l]["k"], 0).numpy().transpose(1, 0, 2)   # [2, T, 256]
        assert np.abs(kf[ai] - ref).max() <= 0.05 * max(1.0, np.abs(ref).max())


def test_batched_lanes_equal_single(eng):
    from oracle.weights import lane_prompt_ids
    from qwen35 import State
    B = 70        # > 64 lanes: batched GEMMs and the whole-head GDN blocks, vs the batch-1 path
    prompts = [lane_prompt_ids(0, b, 5 + (3 * b) % 11) for b in range(B)]
    sb = State(eng, B, 256)
    y = [sb.prefill(b, prompts[b]) for b in range(B)]
    seqb = [[t] for t in y]
    for _ in range(6):
        out = sb.decode_step([s[-1] for s in seqb])
        for b in range(B):
            seqb[b].append(int(out[b]))
    for b in (0, 37, 69):
        s1 = State(eng, 1, 512)
        t = s1.prefill(0, prompts[b])
        seq = [t]
        for _ in range(6):
            seq.append(int(s1.decode_step([seq[-1]])[0]))
        assert seq == seqb[b], b
        assert np.array_equal(s1.read(0, "S"), sb.read(b, "S"))


def test_incremental_equals_batch(eng, golden):
    """G5 (specification/08-state-management.md:111-117): prompt T then decode == prompt T+D."""
    from qwen35 import State
    ids = [int(t) for t in golden["config0_greedy"]["prompt"]]
    a = State(eng, 1, 512)
    a.prefill(0, ids[:20])
    for t in ids[20:31]:
        a.decode_step([t])
    ya, la = a.decode_step([ids[31]], logits=True)
    b = State(eng, 1, 512)
    yb, lb = b.prefill(0, ids, logits=True)
    assert int(ya[0]) == yb
    assert np.array_equal(la[0], lb)
    assert np.array_equal(a.read(0, "S"), b.read(0, "S"))
    assert np.array_equal(a.read(0, "k", 32), b.read(0, "k", 32))


def test_mtp_k2_lossless_and_oracle(eng, golden):
    from qwen35 import State, Forward, greedy_mtp
    g = golden["mtp_k2"]
    ids = [int(t) for t in golden["config0_greedy"]["prompt"]]
    st = State(eng, 1, 512, mtp_k=2, mtp_cap=256)
    f = Forward(eng, st)
    out, stats = greedy_mtp(f, ids, 16, k=2, stop_on_eos=False)
    plain = Forward(eng, State(eng, 1, 512)).greedy(ids, len(out) - 1, stop_on_eos=False)
    assert out == plain[:len(out)]
    assert stats["drafted"] == 2 * stats["bonus"]
    # the reference's greedy_mtp (batched and sequential verify) emits the plain greedy ids,
    # so its ids are golden config-0 rows: the engine's rounds equal them up to the first
    # divergence, which must be at a row the reference prices as a near-tie
    for key in ("batch_tokens", "steps_tokens"):
        ref = [int(t) for t in g[key]]
        n = min(len(out), len(ref))
        agree = next((i for i in range(n) if out[i] != ref[i]), n)
        print(f"mtp k=2: {agree}/{n} ids equal the reference's greedy_mtp ({key}); stats {stats}", flush=True)
        if agree < n:
            assert _golden_near_tie(golden, agree), (key, agree)
        else:
            assert n == min(len(out), 17)


def test_mtp_draft_vs_oracle(eng, oracle_weights, golden):
    from oracle import model
    from qwen35 import State
    ids = [int(t) for t in golden["config0_greedy"]["prompt"]]
    st = State(eng, 1, 512, mtp_k=2, mtp_cap=64)
    y0 = st.prefill(0, ids)
    d, xd, lg = st.mtp_draft([y0], [len(ids) + 1], 0, logits=True)
    f = model.Forward(oracle_weights)
    normed = f.prefill(ids)
    m = model.MTPDraft(oracle_weights)
    dd = {}
    rd, rxd = m.draft(y0, normed[-1:], len(ids) + 1, dd)
    ref = dd["logits"].float().numpy()
    assert np.abs(lg[0] - ref).max() <= LOGIT_MAX
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > GAP:
        assert int(d[0]) == rd
    xdf = (xd[0].astype(np.uint32) << 16).view(np.float32)
    assert np.abs(xdf - rxd[0].float().numpy()).max() <= LOGIT_MAX


def test_graph_replay_equals_eager(eng):
    """hipGraph-captured decode steps, replayed with eager work in between, give the
    same tokens, logits and state as eager launches."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import State
    prompts = [lane_prompt_ids(0, 100 + b, 7) for b in range(3)]
    res = {}
    for mode in (0, 1):
        eng.set_option("graph", mode)
        st = State(eng, 3, 512)
        toks = [st.prefill(b, prompts[b]) for b in range(3)]
        lg_all, tk_all = [], []
        for step in range(5):
            out, lg = st.decode_step(toks, logits=True)
            toks = [int(t) for t in out]
            tk_all.append(toks)
            lg_all.append(lg)
            if mode == 1:            # eager work between replays
                scratch = State(eng, 1, 64)
                scratch.prefill(0, prompts[0][:3])
                scratch.close()
        res[mode] = (tk_all, lg_all, st.read(1, "S"))
        st.close()
    eng.set_option("graph", 0)
    assert res[0][0] == res[1][0]
    for a, b in zip(res[0][1], res[1][1]):
        assert np.array_equal(a, b)
    assert np.array_equal(res[0][2], res[1][2])


def test_one_row_partials_equal_epilogue_add(eng):
    """One-row bodies: the 1024-wide GEMVs leaving k-block chains that the next norm GEMM folds
    into the residual (and the final add+norm) give the same bits as the residual add in the
    GEMV epilogue: tokens, full logits and state, for a one-token prompt and decode steps."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import State
    ids = lane_prompt_ids(3, 0, 9)
    res = {}
    for mode in (0, 1):
        eng.set_option("b1_partials", mode)
        st = State(eng, 1, 512)
        y, lg0 = st.prefill(0, ids[:1], logits=True)
        st.prefill(0, ids[1:])
        toks, lgs = [], [lg0]
        t = int(y)
        for _ in range(4):
            out, lg = st.decode_step([t], logits=True)
            t = int(out[0])
            toks.append(t)
            lgs.append(lg[0])
        res[mode] = (int(y), toks, lgs, st.read(0, "S"), st.read(0, "k", 16))
        st.close()
    eng.set_option("b1_partials", 1)
    assert res[0][0] == res[1][0] and res[0][1] == res[1][1]
    for a, b in zip(res[0][2], res[1][2]):
        assert np.array_equal(a, b)
    assert np.array_equal(res[0][3], res[1][3]) and np.array_equal(res[0][4], res[1][4])


@pytest.mark.parametrize("P", [4096, 9000, 32768, 131072])
def test_seeded_state_decode(oracle_weights, P):
    """The benchmark's seeded workload: lanes with N(0,0.1) GDN state and N(0,1) K/V over P
    slots (P = 9000, 32768 and 131072: up to 512 score chunks and 1024 P.V parts, 4x benchmark config 3's
    longest context) decode one step like the oracle
    holding the same state (oracle/seeded.py)."""
    import torch
    from oracle.seeded import seeded_forward
    from qwen35 import Engine, State
    e = Engine(max_rows=16, max_ctx=P + 64, seed=0)
    st = State(e, 2, P + 16)
    st.seed(1, P)
    toks = [1234, 99]
    out, lg = st.decode_step(toks, logits=True)
    for lane in (0, 1):
        f = seeded_forward(oracle_weights, 1, lane, P)
        ref = f.logits(f.decode(toks[lane]))[-1].float().numpy()
        d = np.abs(lg[lane] - ref)
        print(f"seeded P={P} lane {lane}: max|d|={d.max():.4f} mean|d|={d.mean():.5f}", flush=True)
        assert d.max() <= LOGIT_MAX and d.mean() <= LOGIT_MEAN
        top2 = np.sort(ref)[-2:]
        if top2[1] - top2[0] > GAP:
            assert int(out[lane]) == int(ref.argmax())
        S = st.read(lane, "S")
        for gi, l in enumerate([l for l in range(24) if l % 4 != 3]):
            assert np.abs(S[gi] - f.rec[l].numpy()).max() <= 2e-2
    st.close()
    e.close()


def test_split_attention_forms_identical(eng):
    """The split attention path in 4-wave score blocks and dim-quarter P.V blocks gives the
    bits of the one-wave score / 256-thread P.V kernels: a 40-token prompt wave (rows > 1:
    attn_prep + scores), decode steps (prep folded into the scores) past a 128-slot part
    boundary, and an MTP round (3-row verify) -- tokens, logits and state."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import State
    ids = lane_prompt_ids(91, 0, 40)
    res = {}
    for mode in (0, 1):
        eng.set_option("attn_split4", mode)
        st = State(eng, 1, 512, mtp_k=2, mtp_cap=64)
        y, lg0 = st.prefill(0, ids, logits=True)
        toks, lgs = [int(y)], [lg0]
        for _ in range(100):
            out, lg = st.decode_step([toks[-1]], logits=True)
            toks.append(int(out[0]))
            lgs.append(lg[0])
        em = st.mtp_round([toks[-1]], 2)
        res[mode] = (toks, lgs, em, st.read(0, "S"), st.read(0, "k", 140))
        st.close()
    eng.set_option("attn_split4", 1)
    assert res[0][0] == res[1][0] and res[0][2] == res[1][2]
    for a, b in zip(res[0][1], res[1][1]):
        assert np.array_equal(a, b)
    assert np.array_equal(res[0][3], res[1][3]) and np.array_equal(res[0][4], res[1][4])
