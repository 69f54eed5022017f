"""The portable stream: C build == numpy restatement; distribution sanity."""
import numpy as np

from oracle import prng
from oracle.weights import registry, tensor_bits, VOCAB


def test_c_matches_numpy():
    for tid in (0, 1, prng.fnv1a64("model.language_model.embed_tokens.weight")):
        for start in (0, 12345):
            assert np.array_equal(prng.normal_bf16(7, tid, 0.02, 5000, start), prng.normal_bf16_np(7, tid, 0.02, start, 5000))
            assert np.array_equal(prng.normal_f32(7, tid, 0.1, 5000, start), prng.normal_f32_np(7, tid, 0.1, start, 5000))
        assert np.array_equal(prng.uniform(3, tid, 100), prng.uniform_np(3, tid, 0, 100))
        assert np.array_equal(prng.tokens(0, tid, 64, VOCAB), prng.tokens_np(0, tid, 64, VOCAB))


def test_known_values():
    # splitmix64 reference values: mix(0) is the first output of splitmix64 seeded with 0
    assert prng._mix(0) == 0xE220A8397B1DCDAF
    assert prng.fnv1a64("") == 0xCBF29CE484222325
    assert prng.fnv1a64("a") == 0xAF63DC4C8601EC8C


def test_distribution():
    v = prng.normal_f32(0, 99, 1.0, 2_000_000)
    assert abs(v.mean()) < 5e-3 and abs(v.std() - 1.0) < 5e-3
    u = prng.uniform(0, 99, 100000)
    assert u.min() >= 0 and u.max() < 1 and abs(u.mean() - 0.5) < 5e-3


def test_registry_shapes():
    reg = registry()
    assert len(reg) == 335                       # specimpl.py:62 EXPECTED_LOADED
    names = [r[0] for r in reg]
    assert len(set(names)) == len(names)
    a = tensor_bits(0, "model.language_model.layers.0.linear_attn.A_log", (16,), "alog")
    af = (a.astype(np.uint32) << 16).view(np.float32)
    assert (af >= 0).all() and (af <= np.log(16) + 0.02).all()
    d = tensor_bits(0, "model.language_model.layers.0.linear_attn.dt_bias", (16,), "dtbias")
    df = (d.astype(np.uint32) << 16).view(np.float32)
    assert (np.abs(df) <= 1).all()
