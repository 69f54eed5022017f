"""Op-level parity of the GDN gated RMSNorm (engine/kernels_gdn.cpp:525; oracle rmsnorm_gated,
speccheck/specimpl.py:142-147,304-305) and of the SwiGLU product (specimpl.py:400-407) in every
place the engine makes them:
  * the recurrence's fused epilogue, persistent kernel (decode, B > 64) and whole-head kernel
    (MTP verify rows), through q35_op_gdn_step_norm;
  * the out_proj GEMM's batched A producer (B <= 64 lanes, prompt waves), through
    q35_op_gdn_step_norm and q35_op_gemm_a with M > 16;
  * the one-row GEMM's in-register producer (batch 1), through q35_op_gemm_a with M <= 16 and
    an identity weight matrix, so Y = A exactly (one nonzero product per output, exact in f32,
    and a bf16 value survives the bf16 store).
Bar (stated): all forms are bit-identical to each other (one shared f32 reduction tree), and
every element is within 1 bf16 ulp of the oracle's torch-f32 formula on the same inputs (its
mean over 64 values is summed in another order, which can move the final rounding by one
step); at least 99 % of elements are bit-equal to it."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    """|a - b| in bf16 ulps for same-sign bf16 bit patterns (uint16)."""
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    sa, sb = a >> 15, b >> 15
    ma, mb = a & 0x7FFF, b & 0x7FFF
    d = np.where(sa == sb, np.abs(ma - mb), ma + mb)
    return d


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _check(got, ref, what):
    u = _ulps(got, ref)
    eq = float((u == 0).mean())
    print(f"{what}: max {u.max()} ulp, bit-equal {eq * 100:.3f} %", flush=True)
    assert u.max() <= 1, what
    assert eq >= 0.99, what


@pytest.fixture(scope="module")
def eng():
    from qwen35 import Engine
    e = Engine(max_rows=1024, max_ctx=256, seed=0)
    yield e
    e.close()


@pytest.mark.parametrize("B", [1, 64, 1024])
def test_gdn_gated_norm_all_forms(eng, oracle_weights, B):
    import torch
    from oracle import model
    print(f"gated norm B={B}", flush=True)
    p = "model.language_model.layers.0.linear_attn."
    conv_w, A_log, dt_bias = (oracle_weights.p[p + n] for n in ("conv1d.weight", "A_log", "dt_bias"))
    g = torch.Generator().manual_seed(1000 + B)
    proj = torch.randn(B, 8224, generator=g).to(torch.bfloat16)
    gw = (1.0 + 0.25 * torch.randn(128, generator=g)).to(torch.bfloat16)   # a non-trivial norm weight
    S0 = (torch.randn(B, 16, 128, 128, generator=g) * 0.1).float()
    cw, al, db = conv_w.contiguous().cuda(), A_log.contiguous().cuda(), dt_bias.contiguous().cuda()
    dproj, dgw = proj.cuda(), gw.cuda()
    ys, os_ = [], []
    for form in (0, 1):
        S2 = torch.zeros(B, 2, 16, 128, 128, dtype=torch.float32, device="cuda")
        S2[:, 0] = S0.cuda()
        W2 = torch.zeros(B, 2, 3, 6144, dtype=torch.float32, device="cuda")
        o = torch.empty(B, 2048, dtype=torch.float32, device="cuda")
        y = torch.empty(B, 2048, dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()
        eng.op_gdn_step_norm(dproj.data_ptr(), cw.data_ptr(), al.data_ptr(), db.data_ptr(), dgw.data_ptr(),
                             S2.data_ptr(), W2.data_ptr(), o.data_ptr(), y.data_ptr(), B, form)
        ys.append(_bits(y))
        os_.append(o.cpu())
    assert torch.equal(os_[0], os_[1])
    assert np.array_equal(ys[0], ys[1]), "fused epilogue and producer forms differ"
    z = proj[:, 8192 - 2048:8192]                 # z columns of the projection row
    ref = model.rmsnorm_gated(os_[0].reshape(B * 16, 128), z.reshape(B * 16, 128), gw).to(torch.bfloat16)
    _check(ys[0].reshape(-1), _bits(ref).reshape(-1), f"gdn gated norm B={B}")


def _identity_tiled(eng, n):
    import torch
    w = torch.eye(n, dtype=torch.bfloat16, device="cuda")
    wt = torch.empty_like(w)
    torch.cuda.synchronize()
    eng.op_tile_weight(w.data_ptr(), n, n, wt.data_ptr())
    eng.sync()
    return wt


@pytest.mark.parametrize("amode", [1, 2])
def test_gemm_producers_one_row_and_batched(eng, amode):
    """The in-register (M <= 16) and batched (M > 16) A producers give the same bits for the
    same rows, within 1 ulp of the oracle's formula."""
    import torch
    import torch.nn.functional as F
    from oracle import model
    K = 2048 if amode == 2 else 3584
    M = 200
    wt = _identity_tiled(eng, K)
    g = torch.Generator().manual_seed(7 + amode)
    if amode == 2:
        x = (torch.randn(M, K, generator=g) * torch.rand(M, 1, generator=g) * 3).float()
        x2 = torch.randn(M, K, generator=g).to(torch.bfloat16)
        aux = (1.0 + 0.25 * torch.randn(128, generator=g)).to(torch.bfloat16)
        ref = model.rmsnorm_gated(x.reshape(-1, 128), x2.reshape(-1, 128), aux).to(torch.bfloat16).reshape(M, K)
    else:
        x = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16)
        x2 = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16)
        aux = None
        ref = F.silu(x) * x2                       # bf16 silu, bf16 product (specimpl.py:400-407)
    dx, dx2 = x.cuda(), x2.cuda()
    daux = aux.cuda() if aux is not None else None
    outs = {}
    for m in (1, 16, M):
        y = torch.empty(m, K, dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()
        eng.op_gemm_a(wt.data_ptr(), K, K, amode, dx.data_ptr(), K, dx2.data_ptr(), K,
                      daux.data_ptr() if daux is not None else 0, m, y.data_ptr())
        eng.sync()
        outs[m] = _bits(y)
    assert np.array_equal(outs[1], outs[M][:1]) and np.array_equal(outs[16], outs[M][:16])
    _check(outs[M].reshape(-1), _bits(ref).reshape(-1), f"gemm producer amode={amode}")
