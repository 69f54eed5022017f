"""Decode throughput of the MI355X Qwen3.5-0.8B engine (decode tok/s at batch 1 and 256, ctx 4096, with the HBM roofline fraction).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 256] [--ctx 4096]

A step is one greedy decode step of every lane through the full 24-layer tower plus the
tied lm_head and argmax. Lanes carry seeded state (GDN S ~ N(0,0.1) f32, K/V ~ N(0,1) bf16
over `ctx` slots), weights are the seeded random-init bf16 weights; inputs are resident in
HBM before timing. Prints ONE JSON line: `value` is the batch-`--batch` aggregate tok/s;
the batch-1 figures of the same metric are under "batch1".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (REPO, REPO / "qwen3.5-0.8b_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK = 8000.0            # GB/s, MI355X
MFMA_PEAK = 2500.0           # dense bf16 TFLOP/s, MI355X
WEIGHT_BYTES = 1_504_793_280  # bf16 weights streamed per pass (text tower + tied E)
S_BYTES = 18 * 16 * 128 * 128 * 4
WIN_BYTES = 18 * 3 * 6144 * 4
KV_BYTES_PER_SLOT = 6 * 2 * 2 * 256 * 2   # K and V, 6 layers, 2 kv heads
FAC_ROW_BYTES = 16 * 264 * 4              # one pending GDN row of one layer: k~ | dv | gamma per head
FAM = {"gemm": 1, "lm_head": 2, "gdn": 3, "attn": 4}
KERNEL_NAMES = {"attn": "attn_fused", "gdn": "gdn_persist", "lm_head": "gemm_lmhead3 (tied lm_head)",
                "gemm": "projection / MLP GEMMs"}
# HBM bytes per launch from an earlier rocprofv3 FETCH_SIZE / WRITE_SIZE run (not this run), each
# scaled by what the same counter reads for a 1 GiB copy (FETCH x2.0, WRITE x1.0); the runs and
# the calibration are in the file named by TRAFFIC_SOURCE.
TRAFFIC_SOURCE = "profiles/hbm_traffic_decode_b256_ctx4096.md"
MEASURED_TRAFFIC = {
    ("attn", 256, 4096): (1057685.1 * 2.0 + 1024.0 * 1.0) * 1024,                        # attn_fused
    ("gdn", 256, 4096): (146563.0 * 2.0 + 90236.8 * 1.0) * 1024,    # gdn_persist, gdn_defer 3 (4-step average)
    ("lm_head", 256, 4096): (250420.7 * 2.0 + 2048.0 * 1.0) * 1024,                       # gemm_lmhead3
    # projection / MLP family, the average launch of a step: 24 gate|up (gemm_wide64), 18 in_proj
    # (gemm_pre), 6 qkv (gemm_wide64), 24 down, 24 out/o (FETCH x2 + WRITE per launch of each, KiB)
    ("gemm", 256, 4096): (24 * (9271.0 * 2 + 1792.0) + 18 * (10334.5 * 2 + 4116.2) + 6 * (7220.0 * 2 + 2560.0)
                          + 24 * (4521.0 * 2 + 14336.0) + 24 * (2601.0 * 2 + 8192.0)) / 96 * 1024,
}


def gdn_lane_layer_bytes(d: int) -> float:
    """Algorithmic bytes of one lane's GDN layer per decode step, averaged over the deferral
    cycle of d + 1 steps (engine option gdn_defer = d): the 1 MiB state is read every step and
    written once per cycle; the steps in between write one pending factor row and read the rows
    pending before them (d / 2 on average); plus window r+w, qkv/z/b/a in, o (f32) and y (bf16) out."""
    s = (1 << 20) * (1 + 1 / (d + 1)) + FAC_ROW_BYTES * (d / 2 + d / (d + 1))
    return s + 2 * 73728 + 8224 * 2 + 2048 * 4 + 2048 * 2


def step_bytes(B: int, L: int, d: int) -> int:
    """Algorithmic HBM bytes of one decode step over B lanes at context L."""
    return int(WEIGHT_BYTES + B * (18 * gdn_lane_layer_bytes(d) + KV_BYTES_PER_SLOT * (L + 1)))


def family_bytes(fam: str, B: int, L: int, d: int = 0) -> int:
    """Algorithmic bytes of all launches of one kernel family in one decode step."""
    if fam == "gdn":
        return int(18 * B * gdn_lane_layer_bytes(d))
    if fam == "attn":      # attention core per layer: K and V of L+1 slots, f32 q, bf16 gate in, output
        return 6 * B * (2048 * (L + 1) + 8 * 256 * 4 + 2048 * 2 + 2048 * 2)
    if fam == "lm_head":   # E once, A rows, one (max, index) partial per row and column stream
        return 248320 * 1024 * 2 + B * (1024 * 2 + 128 * 8)
    if fam == "gemm":      # all projection + MLP GEMMs: weights once + activations
        w = WEIGHT_BYTES - 248320 * 1024 * 2 - 24 * 2048 - 1024 * 2
        act = B * 24 * 2 * (1024 + 8224 + 2048 + 1024 + 1024 + 7168 + 7168 + 1024)
        return w + act
    raise ValueError(fam)


def family_flops(fam: str, B: int) -> int:
    """Dense GEMM FLOPs of one decode step's launches of a family (2 per multiply-add)."""
    if fam == "lm_head":
        return 2 * B * 248320 * 1024
    w = (WEIGHT_BYTES - 248320 * 1024 * 2 - 24 * 2048 - 1024 * 2) // 2    # projection + MLP weights
    return 2 * B * w


def run_decode(eng, B: int, ctx: int, steps: int, warmup: int, kprof: str | None):
    import numpy as np
    import torch
    from qwen35 import State
    st = State(eng, B, ctx + steps + warmup + 8)
    st.seed(1, ctx)
    rng = np.random.default_rng(0)
    tok = rng.integers(0, 248320, size=B).astype(np.int32)
    for _ in range(warmup):
        tok = st.decode_step(tok)
    if kprof:                       # timed with per-kernel events: launched eagerly
        eng.set_option("kprof", FAM[kprof])
    eng.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.timer_begin()
    for _ in range(steps):
        tok = st.decode_step(tok)
    ev_ms = eng.timer_end()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kt = None
    if kprof:
        kt = eng.kprof_read()
        eng.set_option("kprof", 0)
    st.close()
    return wall, ev_ms / 1e3, kt


def run_prefill(eng, n: int, reps: int = 2):
    """Prompt of n random ids into one lane (waves of eng.max_rows rows; the GDN layers take the
    chunked form, config 2's T = 4096 case). Returns the best of `reps` timed passes."""
    import numpy as np
    from qwen35 import State
    ids = np.random.default_rng(0).integers(0, 248320, n).astype(np.int32)
    st = State(eng, 1, n + 64)
    st.prefill(0, ids[:64])            # warm: kernels loaded, graphs of the decode path untouched
    st.reset()
    best = None
    for _ in range(reps):
        eng.sync()
        t0 = time.perf_counter()
        st.prefill(0, ids)
        eng.sync()
        dt = time.perf_counter() - t0
        st.reset()
        best = dt if best is None else min(best, dt)
    st.close()
    return {"tokens": n, "ms": round(best * 1e3, 2), "tok_s": round(n / best, 1), "wave_rows": eng.max_rows}


def run_prefill_lanes(eng, B: int, n: int, reps: int = 2):
    """Prompts of n random ids into each of B lanes through shared body passes
    (q35_prefill_lanes). Returns the best of `reps` timed passes."""
    import numpy as np
    from qwen35 import State
    rng = np.random.default_rng(0)
    prompts = [rng.integers(0, 248320, n).astype(np.int32) for _ in range(B)]
    st = State(eng, B, n + 64)
    st.prefill_lanes([p[:4] for p in prompts])     # warm
    best = None
    for _ in range(reps):
        st.reset()
        eng.sync()
        t0 = time.perf_counter()
        st.prefill_lanes(prompts)
        eng.sync()
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    st.close()
    return {"lanes": B, "tokens_per_lane": n, "ms": round(best * 1e3, 2), "tok_s": round(B * n / best, 1),
            "max_rows": eng.max_rows}


def run_mtp(eng, B: int, ctx: int, rounds: int, warmup: int, seed: int = 1, k: int = 2):
    """Config 4: B seeded lanes at context ctx, each round = k MTP drafts + a (k+1)-row verify
    with greedy accept and rollback (q35_mtp_round). Returns emitted tokens/s and accept stats."""
    import numpy as np
    import torch
    from qwen35 import State
    st = State(eng, B, ctx + 3 * (rounds + warmup) + 16, mtp_k=2, mtp_cap=2 * (rounds + warmup) + 16)
    st.seed(seed, ctx)
    tok = np.random.default_rng(seed).integers(0, 248320, size=B).astype(np.int32)
    tok = st.decode_step(tok)             # one plain step: sets each lane's last hidden row
    stats = np.zeros(4, np.int64)
    for _ in range(warmup):
        em = st.mtp_round(tok, k, stats=stats)
        tok = np.array([e[-1] for e in em], np.int32)
    stats[:] = 0
    eng.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    emitted = 0
    for _ in range(rounds):
        em = st.mtp_round(tok, k, stats=stats)
        emitted += sum(len(e) for e in em)
        tok = np.array([e[-1] for e in em], np.int32)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    st.close()
    return {"tok_s": round(emitted / wall, 2), "ms_per_round": round(wall / rounds * 1e3, 3),
            "accept_rate": round(float(stats[1]) / max(int(stats[0]), 1), 4),
            "tokens_per_round_per_lane": round(emitted / rounds / B, 3), "lanes": B, "k": k, "seed": seed}


def run_mtp_adaptive(eng, B: int, ctx: int, turns: int, cost_k1: float = 0.0, cost_k2: float = 0.0):
    """Config 4 with the adaptive depth policy (engine/mtp_adaptive.h) per lane: every turn runs
    each lane at its policy's depth (q35_mtp_adaptive_step), each round billed at the round costs
    measured on this GPU (cost_k1 / cost_k2 plain steps). With random-init weights no draft is
    accepted, so every lane demotes after 16 rounds and abandons after 24 more; reported are the
    whole run's emitted tok/s, the steady state after abandonment and the turn of each depth
    change (the first and last lane to change)."""
    import numpy as np
    import torch
    from qwen35 import MtpPolicy, State
    st = State(eng, B, ctx + 3 * turns + 16, mtp_k=2, mtp_cap=2 * turns + 16)
    st.seed(1, ctx)
    tok = st.decode_step(np.random.default_rng(1).integers(0, 248320, size=B).astype(np.int32))
    pol = [MtpPolicy(2, cost_k1, cost_k2) for _ in range(B)]
    eng.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    emitted, t_abandon, e_abandon, depth_turns = 0, None, 0, {0: 0, 1: 0, 2: 0}
    prev = np.full(B, 2)
    changes = {}                    # "2->1" / "1->0": [first turn, last turn, lanes]
    for t in range(turns):
        em, dep = st.mtp_adaptive_step(tok, pol)
        emitted += sum(len(e) for e in em)
        for d in dep:
            depth_turns[int(d)] += 1
        for a, b in ((2, 1), (1, 0)):
            hit = int(((prev == a) & (dep == b)).sum())
            if hit:
                c = changes.setdefault(f"{a}->{b}", [t, t, 0])
                c[1], c[2] = t, c[2] + hit
        prev = np.asarray(dep).copy()
        tok = np.array([e[-1] for e in em], np.int32)
        if t_abandon is None and (dep == 0).all():
            t_abandon, e_abandon, n_abandon = time.perf_counter(), emitted, t
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    st.close()
    steady = None
    if t_abandon is not None and t_abandon < t0 + wall and turns - n_abandon > 1:
        steady = round((emitted - e_abandon) / (t0 + wall - t_abandon), 2)
    return {"tok_s_whole_run": round(emitted / wall, 2), "tok_s_after_abandon": steady, "turns": turns,
            "lane_turns_at_depth": {str(k): v for k, v in depth_turns.items()}, "lanes": B,
            "depth_changes": {k: {"first_turn": v[0], "last_turn": v[1], "lanes": v[2]} for k, v in changes.items()},
            "round_costs": {"k1": cost_k1, "k2": cost_k2}}


def run_mtp_accepting(eng, B: int, ctx: int, rounds: int, d: int = 7):
    """MTP k = 2 rounds with weights reshaped so drafts accept (final norms keep one hidden
    dimension d, embedding rows 248046 / 1000 get +-8 there: every greedy pick is one of the two
    by the sign of x_d, as in the accept tests). The same work per round as run_mtp; the
    weights are restored afterwards. Returns emitted tok/s, the plain step rate on the same
    weights and the accept rate."""
    import numpy as np
    emb = "model.language_model.embed_tokens.weight"
    names = (emb, "model.language_model.norm.weight", "mtp.norm.weight")
    saved = {n: eng.read_tensor(n, 248320 * 1024 if n == emb else 1024) for n in names}
    E = saved[emb].reshape(248320, 1024).copy()
    E[248046, d] = 0x4100
    E[1000, d] = 0xC100
    nw = np.full(1024, 0xBF80, np.uint16)
    nw[d] = 0x4040
    try:
        eng.load_tensor(emb, E.reshape(-1))
        del E
        for n in names[1:]:
            eng.load_tensor(n, nw)
        # a lane's drafts agree or not depending on its seeded state (73 % of 256 lanes do);
        # with one lane, the first of a few state seeds whose drafts agree in a short probe
        seed = 1
        if B == 1:
            for sd in range(1, 9):
                if run_mtp(eng, 1, ctx, 3, 0, sd)["accept_rate"] > 0:
                    seed = sd
                    break
        res = run_mtp(eng, B, ctx, rounds, 1, seed)
        wall, _, _ = run_decode(eng, B, ctx, rounds, 1, None)
        res["plain_tok_s_same_weights"] = round(B * rounds / wall, 2)
        res["speedup_vs_plain"] = round(res["tok_s"] / res["plain_tok_s_same_weights"], 4)
        return res
    finally:
        for n in names:
            eng.load_tensor(n, saved[n])


def cpu_baseline(ctx: int, budget_s: float = 6.0, runs: int = 3):
    """The torch-CPU oracle (restatement of the reference's specimpl.py path) decoding lane 0
    of the same seeded workload on the host cores: the median tok/s of `runs` timed runs of
    about budget_s each (the baseline protocol: median of 3), continuing one greedy sequence."""
    import statistics
    import torch
    from oracle.seeded import seeded_forward
    from oracle.weights import WeightDict
    torch.set_grad_enabled(False)
    f = seeded_forward(WeightDict(0), 1, 0, ctx)
    tok, total = 1234, 0
    f.decode(tok)                      # warm
    rates = []
    for _ in range(runs):
        n = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget_s or n < 2:
            tok = int(f.logits(f.decode(tok))[-1].argmax())
            n += 1
        rates.append(n / (time.perf_counter() - t0))
        total += n
    return statistics.median(rates), torch.get_num_threads(), total, rates


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--b1-steps", type=int, default=100)
    ap.add_argument("--kprof", default="all", choices=list(FAM) + ["none", "all"],
                    help="kernel families timed with per-launch HIP events (separate eager passes)")
    ap.add_argument("--kprof-steps", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mtp-rounds", type=int, default=5, help="config 4 (MTP k=2) rounds; 0 skips it")
    ap.add_argument("--adaptive-turns", type=int, default=60, help="config 4 turns with the adaptive depth policy")
    ap.add_argument("--prefill-len", type=int, default=4096, help="one-lane prompt prefill length; 0 skips it")
    ap.add_argument("--prefill-rows", type=int, default=2048, help="prompt wave rows (the engine's max_rows)")
    ap.add_argument("--eager", action="store_true", help="launch kernels eagerly (no hipGraph)")
    ap.add_argument("--gdn-defer", type=int, default=3,
                    help="engine option gdn_defer: decode steps a GDN state update stays pending (0: written every step)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="run one 1 GiB device-to-device torch copy first (counter calibration: "
                         "FETCH_SIZE/WRITE_SIZE of a known-size copy)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: lanes are independent sequences, so more GPUs would "
              "each run their own B/N lanes with no collective; multi-GPU runs are not part of "
              "this build.", file=sys.stderr)
        sys.exit(2)
    import torch
    from qwen35 import Engine
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    B, L = args.batch, args.ctx
    if args.calib_copy:
        src = torch.empty(1 << 29, dtype=torch.float16, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    eng = Engine(max_rows=max(3 * B, 64, args.prefill_rows),
                 max_ctx=L + max(args.steps, args.b1_steps, 3 * args.adaptive_turns, 12 * args.mtp_rounds) + args.warmup + 64,
                 seed=0,
                 use_graph=not args.eager)
    eng.set_option("gdn_defer", args.gdn_defer)
    # timed value: graph replay, no per-kernel events
    wall, ev_s, _ = run_decode(eng, B, L, args.steps, args.warmup, None)
    ms = wall / args.steps * 1e3
    value = B * args.steps / wall
    wall1, ev1, kt1 = run_decode(eng, 1, L, args.b1_steps, args.warmup, None)
    ms1 = wall1 / args.b1_steps * 1e3
    gbs = step_bytes(B, L, args.gdn_defer) / (ms / 1e3) / 1e9
    gbs1 = step_bytes(1, L, args.gdn_defer) / (ms1 / 1e3) / 1e9
    # kernel rooflines: short eager passes with HIP events around each launch of one family
    rooflines = {}
    fams = [] if args.kprof == "none" else ([args.kprof] if args.kprof != "all" else ["attn", "gdn", "lm_head", "gemm"])
    for kp in fams:
        _, _, kt = run_decode(eng, B, L, args.kprof_steps, 1, kp)
        if kt is None or kt[1] <= 0:
            continue
        per_launch_ms = kt[0] / kt[1]
        launches_per_step = kt[1] / args.kprof_steps
        byt = family_bytes(kp, B, L, args.gdn_defer) / launches_per_step
        ach = byt / (per_launch_ms / 1e3) / 1e9
        rooflines[kp] = {"kernel": KERNEL_NAMES[kp], "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK,
                         "unit": "GB/s", "frac": round(ach / HBM_PEAK, 4), "traffic": MEASURED_TRAFFIC.get((kp, B, L)),
                         "traffic_source": TRAFFIC_SOURCE if (kp, B, L) in MEASURED_TRAFFIC else None,
                         "bytes_per_launch": int(byt), "avg_launch_us": round(per_launch_ms * 1e3, 2),
                         "launches_per_step": launches_per_step,
                         "us_per_step": round(kt[0] / args.kprof_steps * 1e3, 2)}
        if kp in ("lm_head", "gemm"):   # also priced against dense bf16 MFMA
            tf = family_flops(kp, B) / launches_per_step / (per_launch_ms / 1e3) / 1e12
            rooflines[kp].update({"achieved_tflops": round(tf, 1), "mfma_peak_tflops": MFMA_PEAK,
                                  "mfma_frac": round(tf / MFMA_PEAK, 4)})
    # the dominant kernel family: the largest measured share of the step
    dominant = max(rooflines, key=lambda k: rooflines[k]["us_per_step"]) if rooflines else None
    roof = rooflines.get(dominant)
    mtp = None
    if args.mtp_rounds > 0:
        mtp = run_mtp(eng, B, L, args.mtp_rounds, 1)
        mtp["round_cost_steps"] = round(mtp["ms_per_round"] / ms, 4)
        mk1 = run_mtp(eng, B, L, args.mtp_rounds, 1, k=1)
        mk1["round_cost_steps"] = round(mk1["ms_per_round"] / ms, 4)
        m1 = run_mtp(eng, 1, L, 4 * args.mtp_rounds, 2)
        m1["round_cost_steps"] = round(m1["ms_per_round"] / ms1, 4)
        m1k1 = run_mtp(eng, 1, L, 4 * args.mtp_rounds, 2, k=1)
        m1k1["round_cost_steps"] = round(m1k1["ms_per_round"] / ms1, 4)
        mtp = {"b%d" % B: mtp, "b%d_k1" % B: mk1, "b1": m1, "b1_k1": m1k1,
               "adaptive_b%d" % B: run_mtp_adaptive(eng, B, L, args.adaptive_turns, mk1["round_cost_steps"],
                                                    mtp["round_cost_steps"]),
               "note": "random-init weights: the drafter almost never agrees with the target"}
        mtp["accepting_b%d" % B] = run_mtp_accepting(eng, B, L, args.mtp_rounds)
        mtp["accepting_b1"] = run_mtp_accepting(eng, 1, L, 4 * args.mtp_rounds)
    pre = run_prefill(eng, args.prefill_len) if 0 < args.prefill_len <= eng.max_ctx - 64 else None
    if pre is not None:
        # the same prompt byte-identical to token-by-token feeding (prompt_exact): its price
        eng.set_option("prompt_exact", 1)
        pre["exact"] = run_prefill(eng, args.prefill_len, reps=1)
        eng.set_option("prompt_exact", 0)
        pre["lanes"] = run_prefill_lanes(eng, B, 64)
    cpu = None
    if not args.no_cpu:
        tps, thr, n, rates = cpu_baseline(L)
        cpu = {"value": round(tps, 3), "unit": "tok/s", "cores": thr, "nproc": len(os.sched_getaffinity(0)), "kind": "port",
               "runs": [round(r, 3) for r in rates],
               "sample": f"oracle (torch CPU restatement of speccheck/specimpl.py) greedy decode of lane 0 "
                         f"of this workload (seeded state, ctx {L}), batch 1: median of {len(rates)} timed runs "
                         f"of ~6 s, {n} tokens in all"}
    out = {"metric": "decode tok/s at batch 1 and 256 (ctx 4k); achieved HBM GB/s vs 8 TB/s peak",
           "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "bf16", "data": "synthetic (seeded random-init weights and state)",
           "config": {"workload": f"decode_b{B}_ctx{L}", "model": "Qwen3.5-0.8B text tower", "global_batch": B,
                      "seq_len": L, "parallelism": "none (1 GPU)", "gdn_defer": args.gdn_defer},
           "hbm_gbs_step": round(gbs, 1), "hbm_frac_step": round(gbs / HBM_PEAK, 4),
           # the same step priced with the state written back every step (gdn_defer 0), as the
           # reference's decode does: the bytes a non-deferring engine must move for this output
           "hbm_frac_step_writeback_every_step": round(step_bytes(B, L, 0) / (ms / 1e3) / 1e9 / HBM_PEAK, 4),
           "event_ms_per_step": round(ev_s / args.steps * 1e3, 4),
           "batch1": {"tok_s": round(args.b1_steps / wall1, 2), "ms_per_step": round(ms1, 4),
                      "hbm_gbs": round(gbs1, 1), "hbm_frac": round(gbs1 / HBM_PEAK, 4),
                      "bytes_per_token": step_bytes(1, L, args.gdn_defer)},
           "mtp_k2": mtp, "prefill": pre, "roofline": roof,
           "kernel_rooflines": {k: v for k, v in rooflines.items() if k != dominant}, "cpu_baseline": cpu}
    print(json.dumps(out))


if __name__ == "__main__":
    main()
