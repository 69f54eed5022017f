"""Flash-form prompt-wave attention (attn_prompt: one lane's wave of >= 64 rows, 16 rows x 4
heads per block, QK^T and P.V on MFMA, online softmax) against a float64 restatement of the
reference's attention (speccheck/specimpl.py:370-397: scores q.K / 16 in f32, softmax,
weights rounded to bf16, P.V, bf16 output times bf16(sigmoid(gate))) on the engine's own
last-layer inputs: post-rope q (scratch "q"), the K/V cache of layer 23 and the gate half of
the projection rows. Cases: one-wave prompts whose row count is and is not a multiple of
16, and a second wave continuing after a prefix (slots start above 0).

Tolerance (stated): the kernel rounds the unnormalised weights e^(s - m) to bf16 and divides
by the sum afterwards, the reference rounds the normalised weights, so each weight carries
a different bf16 rounding: the kernel's weight bf16(e_t) / sum_s bf16(e_s) is off the exact
softmax weight by at most 2^-9 for its own rounding plus 2^-9 for the normaliser's (a
weighted mean of the same roundings), the reference's by 2^-9 -- 3 x 2^-9 of each weight
apart -- and the bf16 output may land one rounding step away: every element within 2 bf16
ulps of the reference value plus 3 x 2^-9 sum_t p_t |v_t| sigmoid(gate) (the weight-rounding
bound, which decides outputs that cancel to near zero), and mean |d| <= 2^-10 (measured
~4.5e-4 on outputs up to ~5). The one-row kernels
meet the same bound on the same inputs (checked in the test; they round like the
reference, mean |d| ~1e-6), and the full-model prompt logits
stay within the engine-vs-oracle tolerance (test_chunked_prefill_vs_oracle_chunk_form runs
its 600-token prompt through this kernel)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REL_W, MEAN_D = 3 * 2.0 ** -9, 2.0 ** -10


def _bf(a):
    """float64 -> nearest bf16 value (round to nearest even), as float64."""
    f = np.asarray(a, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def _u16f(x):
    return (np.asarray(x, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _reference(q, K, V, gate, slots):
    """q [T][8][256] f32, K/V [2][S][256] bf16 values, gate [T][8][256] bf16 values."""
    T = q.shape[0]
    out = np.empty((T, 8, 256))
    mag = np.empty((T, 8, 256))          # sum_t p_t |v_t| * gate: scale of a weight-rounding error
    for r in range(T):
        s = slots[r]
        for h in range(8):
            j = h // 4
            sc = (K[j, : s + 1] @ q[r, h].astype(np.float64)) / 16.0
            p = np.exp(sc - sc.max())
            p = _bf(p / p.sum())
            o = _bf(p @ V[j, : s + 1])
            g = _bf(1.0 / (1.0 + np.exp(-gate[r, h])))
            out[r, h] = _bf(o * g)
            mag[r, h] = (p @ np.abs(V[j, : s + 1])) * g
    return out, mag


def _run(eng, pre, n, mode):
    from oracle.weights import lane_prompt_ids
    from qwen35 import State
    eng.set_option("attn_prompt", mode)
    st = State(eng, 1, 2048)
    if pre:
        st.prefill(0, lane_prompt_ids(8, 0, pre))
    st.prefill(0, lane_prompt_ids(8, 1, n))
    q = eng.read_scratch("q", (n, 8, 256), np.float32)
    aout = _u16f(eng.read_scratch("aout", (n, 2048), np.uint16)).reshape(n, 8, 256)
    proj = eng.read_scratch("proj", (n, 5120), np.uint16)
    kv_k = st.read(0, "k", pre + n)[5]
    kv_v = st.read(0, "v", pre + n)[5]
    st.close()
    eng.set_option("attn_prompt", 1)
    gate = _u16f(proj[:, :4096].reshape(n, 8, 512)[:, :, 256:])
    return q, _u16f(kv_k), _u16f(kv_v), gate, aout


@pytest.fixture(scope="module")
def eng():
    from qwen35 import Engine
    e = Engine(max_rows=512, max_ctx=2048, seed=0)
    yield e
    e.close()


@pytest.mark.parametrize("pre,n", [(0, 64), (0, 333), (0, 512), (300, 100)])
def test_prompt_attention_vs_float64(eng, pre, n):
    print(f"attn_prompt pre={pre} n={n}", flush=True)
    slots = list(range(pre, pre + n))
    for mode in (1, 0):
        q, K, V, gate, aout = _run(eng, pre, n, mode)
        ref, mag = _reference(q, K, V, gate, slots)
        d = np.abs(aout - ref)
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -40))) - 7)
        print(f"  mode {mode}: max |d| {d.max():.3g}, mean |d| {d.mean():.3g}, max |ref| {np.abs(ref).max():.3g}",
              flush=True)
        assert np.isfinite(aout).all()
        assert (d <= 2 * ulp + REL_W * mag).all() and d.mean() <= MEAN_D, (mode, d.max(), d.mean())


def _untile(buf, rows, K):
    """Rows [rows][K] of a buffer in the GEMMs' tiled fragment layout (16-row tiles; within a
    tile and 256-wide k-block, step s = (k % 256) / 8 % 8, lane = 16 (k % 256 / 64) + row % 16,
    8 consecutive k per lane): the layout a prompt wave of >= 1,024 rows leaves its attention
    output in for the many-row o_proj."""
    r = np.arange(rows)[:, None]
    k = np.arange(K)[None, :]
    kk = k & 255
    lane = (kk >> 6) * 16 + (r & 15)
    off = ((((r >> 4) * (K >> 8) + (k >> 8)) * 8 + ((kk >> 3) & 7)) * 64 + lane) * 8 + (kk & 7)
    return buf.reshape(-1)[off]


def test_prompt_attention_long_context_sampled_rows():
    """A 2,048-row wave after a 2,000-slot prefix (contexts up to 4,048 slots: 64 K/V tiles,
    the online softmax rescaling across many tiles), checked on 48 sampled rows (every head)
    against the same float64 restatement and bound."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, State
    eng = Engine(max_rows=2048, max_ctx=4160, seed=0)
    try:
        pre, n = 2000, 2048
        st = State(eng, 1, 4160)
        st.prefill(0, lane_prompt_ids(9, 0, pre))
        st.prefill(0, lane_prompt_ids(9, 1, n))
        q = eng.read_scratch("q", (n, 8, 256), np.float32)
        # the 2,048-row wave's o_proj runs in the many-row full-K form: aout is tiled
        aout = _u16f(_untile(eng.read_scratch("aout", (n, 2048), np.uint16), n, 2048)).reshape(n, 8, 256)
        proj = eng.read_scratch("proj", (n, 5120), np.uint16)
        K = _u16f(st.read(0, "k", pre + n)[5])
        V = _u16f(st.read(0, "v", pre + n)[5])
        st.close()
    finally:
        eng.close()
    gate = _u16f(proj[:, :4096].reshape(n, 8, 512)[:, :, 256:])
    rows = np.unique(np.concatenate([[0, 1, 15, 16, 63, 64, n - 1], np.random.default_rng(5).integers(0, n, 41)]))
    ref, mag = _reference(q[rows], K, V, gate[rows], [pre + int(r) for r in rows])
    got = aout[rows]
    d = np.abs(got - ref)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -40))) - 7)
    print(f"  long context: {rows.size} rows, max |d| {d.max():.3g}, mean |d| {d.mean():.3g}", flush=True)
    assert np.isfinite(got).all()
    assert (d <= 2 * ulp + REL_W * mag).all() and d.mean() <= MEAN_D, (d.max(), d.mean())


def test_prompt_attention_full_odd_capacity():
    """A lane whose capacity (1,000 slots: not a multiple of the 64-slot tiles) is filled by
    one 999-row wave: the last K/V tile is partial and the padded tail of the cache is never
    read into a weight; every row checked."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, State
    eng = Engine(max_rows=1024, max_ctx=1024, seed=0)
    try:
        n = 999
        st = State(eng, 1, 1000)
        st.prefill(0, lane_prompt_ids(10, 0, n))
        q = eng.read_scratch("q", (n, 8, 256), np.float32)
        aout = _u16f(eng.read_scratch("aout", (n, 2048), np.uint16)).reshape(n, 8, 256)
        proj = eng.read_scratch("proj", (n, 5120), np.uint16)
        K = _u16f(st.read(0, "k", n)[5])
        V = _u16f(st.read(0, "v", n)[5])
        st.close()
    finally:
        eng.close()
    gate = _u16f(proj[:, :4096].reshape(n, 8, 512)[:, :, 256:])
    ref, mag = _reference(q, K, V, gate, list(range(n)))
    d = np.abs(aout - ref)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -40))) - 7)
    print(f"  odd capacity: max |d| {d.max():.3g}, mean |d| {d.mean():.3g}", flush=True)
    assert np.isfinite(aout).all()
    assert (d <= 2 * ulp + REL_W * mag).all() and d.mean() <= MEAN_D, (d.max(), d.mean())


def test_kernel_forms_are_per_engine(eng):
    """A kernel-form switch set on one engine leaves another engine of the process alone: the
    second engine's prompt logits keep the bits of its own (flash-form) kernel."""
    from oracle.weights import lane_prompt_ids
    from qwen35 import Engine, State
    ids = lane_prompt_ids(8, 2, 96)

    def run(e):
        st = State(e, 1, 256)
        y, lg = st.prefill(0, ids, logits=True)
        st.close()
        return y, lg

    y1, l1 = run(eng)
    other = Engine(max_rows=512, max_ctx=2048, seed=0)
    try:
        other.set_option("attn_prompt", 0)
        y0, l0 = run(other)
        y2, l2 = run(eng)
    finally:
        other.close()
    assert y1 == y2 and np.array_equal(l1, l2)
    assert not np.array_equal(l0, l1)    # the one-row kernels round the weights differently
