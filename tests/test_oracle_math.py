"""Pins oracle/model.py's functions against float64 brute force (oracle/ref64.py),
closed forms and invariants, chosen so that a dropped term, a swapped operand or a wrong
index fails (specification/03-05 and their stated invariants)."""
import numpy as np
import torch
import torch.nn.functional as F

from oracle import model, ref64

torch.set_grad_enabled(False)
BF = torch.bfloat16


def bf(x):
    return torch.tensor(np.asarray(x, np.float32)).to(BF)


def ulp_bf16(x):
    x = np.maximum(np.abs(np.asarray(x, np.float64)), 1e-30)
    return 2.0 ** (np.floor(np.log2(x)) - 7)


def test_rmsnorm_zc_vs_f64_and_affine():
    rng = np.random.default_rng(0)
    x = bf(rng.normal(size=(5, 1024)))
    w = bf(rng.normal(size=1024) * 0.1)
    got = model.rmsnorm_zc(x, w).float().numpy()
    ref = ref64.rmsnorm_zc(x.float().numpy(), w.float().numpy())
    assert np.all(np.abs(got - ref) <= ulp_bf16(ref) + 1e-6)
    # (1 + w): w = 0 gives unit RMS, w = 1 gives RMS 2 (a plain-w affine would give 0 and 1)
    for wv, rms in ((0.0, 1.0), (1.0, 2.0)):
        y = model.rmsnorm_zc(x, torch.full((1024,), wv, dtype=BF)).float().numpy()
        assert np.allclose(np.sqrt((y ** 2).mean(-1)), rms, rtol=5e-3)


def test_rmsnorm_gated_vs_f64():
    rng = np.random.default_rng(1)
    o = torch.tensor(rng.normal(size=(6, 128)) * 1e-3, dtype=torch.float32)
    z = bf(rng.normal(size=(6, 128)))
    w = bf(1.0 + rng.normal(size=128) * 0.1)
    got = model.rmsnorm_gated(o, z, w).to(BF).float().numpy()
    ref = ref64.rmsnorm_gated(o.numpy(), z.float().numpy(), w.float().numpy())
    assert np.all(np.abs(got - ref) <= ulp_bf16(ref) + 1e-6)


def test_rope():
    rng = np.random.default_rng(2)
    x = bf(rng.normal(size=(3, 8, 256)))
    pos = torch.tensor([0, 7, 4095])
    cos, sin = model.rope_cs(pos)
    got = model.apply_rope(x, cos, sin).numpy()
    for t, p in enumerate(pos.tolist()):
        ref = ref64.rope(x[t].float().numpy(), p)
        assert np.abs(got[t] - ref).max() <= 2e-3 * max(1.0, abs(p) * 1e-3)
    assert np.array_equal(got[0], x[0].float().numpy())              # position 0 = identity
    assert np.allclose(np.linalg.norm(got, axis=-1), np.linalg.norm(x.float().numpy(), axis=-1), rtol=1e-5)
    assert np.array_equal(got[..., 64:], x[..., 64:].float().numpy())  # dims 64.. pass through


def test_conv_and_window_invariant():
    rng = np.random.default_rng(3)
    T = 5
    raw = bf(rng.normal(size=(T, 6144)))
    C = bf(rng.normal(size=(6144, 1, 4)) * 0.3)
    win = bf(rng.normal(size=(3, 6144)))
    u, nw = model.gdn_conv(raw, C, win)
    ref, rw = ref64.causal_conv(raw.float().numpy(), C.float().numpy().reshape(6144, 4), win.float().numpy())
    sil = ref / (1 + np.exp(-ref))
    assert np.abs(u.float().numpy() - sil).max() <= 0.02 * max(1.0, np.abs(sil).max())
    assert torch.equal(nw, raw[-3:])                                   # window = last 3 raw rows
    _, nw1 = model.gdn_conv(raw[:1], C, win)
    assert torch.equal(nw1, torch.cat([win[1:], raw[:1]]))


def test_gates_closed_form():
    a = bf([-30.0, -1.0, 0.0, 0.5, 19.0, 25.0])
    b = bf([-5.0, 0.0, 5.0, 1.0, -1.0, 2.0])
    A_log = bf([np.log(2.0)] * 6)
    dtb = bf([0.0, 0.5, -0.5, 1.0, 0.5, -3.0])
    g, beta = model.gdn_gates(a, b, A_log, dtb)
    rg, rb = ref64.gates(a.float().numpy(), b.float().numpy(), A_log.float().numpy(), dtb.float().numpy())
    assert np.allclose(g.numpy(), rg, rtol=1e-5) and np.allclose(beta.numpy(), rb, rtol=1e-6)
    A = np.exp(float(A_log[0]))
    assert abs(g.numpy()[4] - (-A * np.log1p(np.exp(19.5)))) < 1e-4   # below 20: log1p(exp(x))
    assert abs(g.numpy()[5] - (-A * 22.0)) < 1e-4                      # above 20: linear


def test_delta_rule_vs_f64_and_invariants():
    rng = np.random.default_rng(4)
    T, H = 6, 3
    q = torch.tensor(rng.normal(size=(T, H, 128)), dtype=torch.float32)
    k = torch.tensor(rng.normal(size=(T, H, 128)), dtype=torch.float32)
    v = torch.tensor(rng.normal(size=(T, H, 128)), dtype=torch.float32)
    qn, kn = model.l2_scale(q, k)
    assert np.allclose(np.linalg.norm(kn.numpy(), axis=-1), 1.0, atol=1e-5)
    assert np.allclose(np.linalg.norm(qn.numpy(), axis=-1), 128 ** -0.5, atol=1e-6)
    g = torch.tensor(-rng.uniform(0, 1, size=(T, H)), dtype=torch.float32)
    beta = torch.tensor(rng.uniform(0, 1, size=(T, H)), dtype=torch.float32)
    S0 = torch.tensor(rng.normal(size=(H, 128, 128)) * 0.1, dtype=torch.float32)
    o, S = model.gdn_recurrent(qn, kn, v, g.exp(), beta, S0.clone())
    ro, rS = ref64.delta_rule(qn.numpy(), kn.numpy(), v.numpy(), g.numpy(), beta.numpy(), S0.numpy())
    assert np.abs(o.numpy() - ro).max() < 1e-4 and np.abs(S.numpy() - rS).max() < 1e-4
    # beta = 0 and g = 0 leave S unchanged and read o = S^T q
    o0, S1 = model.gdn_recurrent(qn, kn, v, torch.ones(T, H), torch.zeros(T, H), S0.clone())
    assert torch.equal(S1, S0)
    assert np.allclose(o0[2].numpy(), np.einsum("hkd,hk->hd", S0.numpy(), qn[2].numpy()), atol=1e-5)


def test_chunk_equals_recurrent():
    rng = np.random.default_rng(5)
    T, H = 100, 2                                        # two chunks, ragged tail
    qn, kn = model.l2_scale(torch.tensor(rng.normal(size=(T, H, 128)), dtype=torch.float32),
                            torch.tensor(rng.normal(size=(T, H, 128)), dtype=torch.float32))
    v = torch.tensor(rng.normal(size=(T, H, 128)), dtype=torch.float32)
    g = torch.tensor(-rng.uniform(0, 0.5, size=(T, H)), dtype=torch.float32)
    beta = torch.tensor(rng.uniform(0, 1, size=(T, H)), dtype=torch.float32)
    S0 = torch.tensor(rng.normal(size=(H, 128, 128)) * 0.1, dtype=torch.float32)
    oc, Sc = model.gdn_chunk_scan(qn, kn, v, g, beta, S0.clone())
    orr, Sr = model.gdn_recurrent(qn, kn, v, g.exp(), beta, S0.clone())
    cos = (oc * orr).sum() / (oc.norm() * orr.norm())
    assert cos > 0.99999 and (Sc - Sr).abs().max() < 1e-3


def test_attention_core_and_single_slot():
    rng = np.random.default_rng(6)
    q = rng.normal(size=256)
    K = rng.normal(size=(37, 256))
    V = rng.normal(size=(37, 256))
    s = torch.tensor(K @ q / 16, dtype=torch.float32)
    p = torch.softmax(s, -1).to(BF)
    got = (p.float().numpy() @ V)
    ref = ref64.attention_row(q, K, V)
    assert np.abs(got - ref).max() < 0.02 * np.abs(V).max()
    # one slot: softmax weight 1 -> output = v exactly
    p1 = torch.softmax(torch.tensor([3.7]), -1).to(BF)
    assert p1.item() == 1.0


def test_argmax_lowest_id_on_ties():
    row = torch.zeros(100, dtype=BF)
    row[[17, 42, 99]] = 3.0
    assert model.argmax_lowest(row) == 17
    row[5] = float("-inf")
    assert model.argmax_lowest(row) == 17


def test_swiglu_exhaustive_bf16():
    """bf16 SiLU over all 65,536 bf16 values: within 1 bf16 ulp of float64 SiLU
    (the policy rounds silu(g) to bf16 before the product, specimpl.py:404-407)."""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(BF)
    x = bits.float().numpy().astype(np.float64)
    fin = np.isfinite(x)
    got = F.silu(bits).float().numpy()[fin]
    ref = (x / (1 + np.exp(-x)))[fin]
    err = np.abs(got - ref) / ulp_bf16(ref)
    assert np.all(err <= 1.0 + 1e-9)
    assert np.mean(err <= 0.5 + 1e-9) > 0.999


def test_bf16_matmul_policy():
    rng = np.random.default_rng(7)
    x = bf(rng.normal(size=(3, 1024)))
    W = bf(rng.normal(size=(64, 1024)) * 0.02)
    got = (x @ W.t()).float().numpy()
    ref = x.double().numpy() @ W.double().numpy().T
    acc = np.abs(x.double().numpy()) @ np.abs(W.double().numpy()).T * 1024 * 2 ** -24
    assert np.all(np.abs(got - ref) <= ulp_bf16(ref) + acc)


def test_incremental_equals_batch(oracle_weights):
    """G5 (specification/08-state-management.md:111-117) on the oracle: prompt T then decode
    equals the longer prompt, tokens equal and logits within bf16 noise."""
    from oracle.weights import prompt_ids
    ids = prompt_ids(0, 12)
    a = model.Forward(oracle_weights)
    a.prefill(ids[:8])
    for t in ids[8:11]:
        a.decode(t)
    la = a.logits(a.decode(ids[11]))[-1].float()
    b = model.Forward(oracle_weights)
    lb = b.logits(b.prefill(ids))[-1].float()
    assert int(la.argmax()) == int(lb.argmax()) or (la.max() - la.topk(2).values[1]) < 0.1
    assert (la - lb).abs().max() < 0.5
