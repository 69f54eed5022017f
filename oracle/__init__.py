"""CPU oracle for the Qwen3.5-0.8B decode path.

TEST INFRASTRUCTURE ONLY. This package is the checker, never the product: only
`tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import it.
The product path (`qwen3.5-0.8b_amd/`) never imports, links or runs anything here and
fails loudly when its HIP library is missing.

Contents
  prng.py / prng.c   portable seeded generator of the synthetic weights and inputs
  weights.py         tensor registry (names, shapes, init) and the weight dict
  model.py           op-for-op torch-CPU restatement of speccheck/specimpl.py and
                     speccheck/mtp.py (the reference's torch CPU path)
  ref64.py           float64 numpy brute-force forms used to pin model.py's math

Pinning status (what checks each function; see tests/test_oracle_*.py):
  rmsnorm_zc, rmsnorm_gated, rope, gdn conv/gates/recurrence, attention, mlp,
  argmax     -> float64 brute force on small shapes + closed-form special cases, and
                bit-exact against tests/golden/ vectors written by importing the
                reference's own specimpl.py in the build container
  gdn_chunk_scan -> chunk == recurrent equivalence (float64) + golden vectors
  Forward / greedy / snapshot / restore -> golden token ids + logits of config 0,
                incremental == batch invariant
  MTPDraft / greedy_mtp -> golden ids + losslessness invariant (verify="steps")
"""
