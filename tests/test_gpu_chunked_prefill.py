"""Chunked (UT-transform, chunk 64) GatedDeltaNet prompt path
(speccheck/specimpl.py:187-235) against the recurrent path of the same engine and against the
oracle's own chunk form (oracle/model.py gdn_chunk_scan).

Tolerances (stated and checked):
  * layer 0 sees identical inputs on both paths: its conv window is bit-identical and its
    f32 state agrees to a relative Frobenius error <= 1e-4 (two association orders of the
    same recurrence; the reference's own gate asks cos >= 0.99999 between the forms)
  * deeper layers and the logits carry the bf16-level divergence of their inputs:
    state relative error <= 6e-2, logits max |d| <= 0.375 and mean |d| <= 0.05, as for
    the other engine-vs-oracle checks
A 512-row wave keeps the engine's chunk boundaries on multiples of 64 from the prompt start,
the oracle's chunking."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_MAX, LOGIT_MEAN = 0.375, 0.05
GDN_LAYERS = [l for l in range(24) if l % 4 != 3]


@pytest.fixture(scope="module")
def eng512():
    import torch
    assert torch.cuda.is_available()
    from qwen35 import Engine
    e = Engine(max_rows=512, max_ctx=2048, seed=0)
    yield e
    e.close()


def _prefill(eng, ids, chunked):
    from qwen35 import State
    eng.set_option("gdn_chunked", 1 if chunked else 0)
    st = State(eng, 1, 2048)
    y, lg = st.prefill(0, ids, logits=True)
    out = (y, lg, st.read(0, "S"), st.read(0, "win"))
    st.close()
    eng.set_option("gdn_chunked", 1)
    return out


@pytest.mark.parametrize("n", [64, 333, 1100])
def test_chunked_equals_recurrent(eng512, n):
    from oracle.weights import lane_prompt_ids
    ids = lane_prompt_ids(7, 0, n)
    print(f"chunked vs recurrent prompt n={n}", flush=True)
    yc, lc, Sc, wc = _prefill(eng512, ids, True)
    yr, lr, Sr, wr = _prefill(eng512, ids, False)
    assert np.array_equal(wc[0], wr[0])
    rel0 = np.linalg.norm(Sc[0] - Sr[0]) / np.linalg.norm(Sr[0])
    assert rel0 <= 1e-4, rel0
    for gi in range(18):
        rel = np.linalg.norm(Sc[gi] - Sr[gi]) / np.linalg.norm(Sr[gi])
        assert rel <= 6e-2, (GDN_LAYERS[gi], rel)
    d = np.abs(lc - lr)
    assert d.max() <= LOGIT_MAX and d.mean() <= LOGIT_MEAN, (d.max(), d.mean())


def test_chunked_prefill_vs_oracle_chunk_form(eng512, oracle_weights):
    from oracle import model
    from oracle.weights import lane_prompt_ids
    n = 600                                  # two waves: 512 + 88 rows
    ids = lane_prompt_ids(11, 0, n)
    f = model.Forward(oracle_weights, gdn_form="chunk")
    normed = f.prefill(ids)                  # final-normed rows [n, 1024] bf16
    ref = f.logits(normed[-1:])[0].float().numpy()
    y, lg, S, w = _prefill(eng512, ids, True)
    d = np.abs(lg - ref)
    assert d.max() <= LOGIT_MAX and d.mean() <= LOGIT_MEAN, (d.max(), d.mean())
    for gi, l in enumerate(GDN_LAYERS):
        r = f.rec[l].numpy()
        rel = np.linalg.norm(S[gi] - r) / np.linalg.norm(r)
        assert rel <= 6e-2, (l, rel)
    r0 = f.rec[0].numpy()
    assert np.linalg.norm(S[0] - r0) / np.linalg.norm(r0) <= 1e-3
