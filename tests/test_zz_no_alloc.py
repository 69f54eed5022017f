"""The allocation-free GDN step (q35_op_gdn_step_noalloc: its lane list in a fixed per-GPU
device array, no hipMalloc / hipFree, asynchronous) against q35_op_gdn_step on the same inputs:
new state, conv window and o bit-identical, on two calls in a row, the second with fewer lanes
(the array keeps the first call's contents), and the size limit refused with an error."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(B, seed):
    import torch
    g = torch.Generator().manual_seed(seed)
    proj = torch.randn(B, 8224, generator=g).to(torch.bfloat16)
    S2 = torch.zeros(B, 2, 16, 128, 128, dtype=torch.float32)
    S2[:, 0] = torch.randn(B, 16, 128, 128, generator=g) * 0.1
    W2 = torch.zeros(B, 2, 3, 6144, dtype=torch.float32)
    W2[:, 0] = torch.randn(B, 3, 6144, generator=g).to(torch.bfloat16).float()
    return proj, S2, W2


def test_noalloc_refuses_another_engine_while_busy(oracle_weights):
    """Two engines on one GPU share the array: while one engine's call is unfinished, the other
    engine's call is refused (it would race); after a sync it runs, and matches."""
    import torch
    from qwen35 import Engine, EngineError
    ea = Engine(max_rows=64, max_ctx=256, seed=None)
    eb = Engine(max_rows=64, max_ctx=256, seed=None)
    try:
        p = "model.language_model.layers.0.linear_attn."
        cw, al, db = (oracle_weights.p[p + n].contiguous().cuda() for n in ("conv1d.weight", "A_log", "dt_bias"))
        B = 4096                     # ~8 GiB of state: a call that runs for milliseconds
        print(f"noalloc two engines B={B}", flush=True)
        proj = torch.randn(B, 8224, device="cuda").to(torch.bfloat16)
        S2 = torch.zeros(B, 2, 16, 128, 128, dtype=torch.float32, device="cuda")
        W2 = torch.zeros(B, 2, 3, 6144, dtype=torch.float32, device="cuda")
        o = torch.empty(B, 2048, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        args = (proj.data_ptr(), cw.data_ptr(), al.data_ptr(), db.data_ptr(), S2.data_ptr(), W2.data_ptr(),
                o.data_ptr())
        ea.op_gdn_step_noalloc(*args, B)
        with pytest.raises(EngineError, match="in use by another engine"):
            eb.op_gdn_step_noalloc(*args, 8)
        ea.op_gdn_step_noalloc(*args, B)          # the same engine: ordered on its stream
        ea.sync()
        eb.op_gdn_step_noalloc(*args, 8)          # the GPU's last call is done: runs
        eb.sync()
    finally:
        ea.close()
        eb.close()


def test_noalloc_gdn_step_equals_allocating_step(oracle_weights):
    import torch
    from qwen35 import Engine, EngineError
    eng = Engine(max_rows=64, max_ctx=256, seed=None)
    try:
        p = "model.language_model.layers.0.linear_attn."
        cw, al, db = (oracle_weights.p[p + n].contiguous().cuda() for n in ("conv1d.weight", "A_log", "dt_bias"))
        for B in (300, 7):            # whole-head persistent kernel, then column-sliced blocks
            print(f"noalloc gdn step B={B}", flush=True)
            proj, S2, W2 = _inputs(B, 11 + B)
            dproj = proj.cuda()
            res = []
            for noalloc in (False, True):
                dS, dW = S2.cuda(), W2.cuda()
                o = torch.full((B, 2048), float("nan"), dtype=torch.float32, device="cuda")
                torch.cuda.synchronize()
                args = (dproj.data_ptr(), cw.data_ptr(), al.data_ptr(), db.data_ptr(), dS.data_ptr(),
                        dW.data_ptr(), o.data_ptr(), B)
                if noalloc:
                    eng.op_gdn_step_noalloc(*args)
                    eng.sync()
                else:
                    eng.op_gdn_step(*args)
                res.append((dS[:, 1].cpu(), dW[:, 1].cpu(), o.cpu()))
            for a, b in zip(*res):
                assert torch.equal(a, b), B
            assert not torch.isnan(res[1][2]).any()
        with pytest.raises(EngineError):
            eng.op_gdn_step_noalloc(dproj.data_ptr(), cw.data_ptr(), al.data_ptr(), db.data_ptr(), 1, 1, 1, 4097)
    finally:
        eng.close()
