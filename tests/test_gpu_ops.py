"""Per-op parity on the GPU through the C ABI: GEMM family and tied lm_head argmax.

Bar: every bf16 output within 1 bf16 ulp of the float64 product of the same bf16 inputs
rounded once (the reference's torch bf16 matmul: f32 accumulate, one rounding); argmax
bit-exact given the engine's own bf16 logits, lowest id on ties."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.fixture(scope="module")
def eng():
    import torch
    assert torch.cuda.is_available()
    from qwen35 import Engine
    e = Engine(max_rows=64, max_ctx=1024, seed=0)
    yield e
    e.close()


@pytest.mark.parametrize("N,K,M", [(16, 256, 1), (6144, 1024, 1), (1024, 2048, 3), (1024, 3584, 16), (512, 1024, 33), (1024, 2048, 200), (8224, 1024, 64)])
def test_gemm_vs_float64(eng, N, K, M):
    import torch
    print(f"gemm N={N} K={K} M={M}", flush=True)
    g = torch.Generator().manual_seed(N + K + M)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16)
    Wd, Xd = W.cuda(), X.cuda()
    Wt = torch.empty_like(Wd)
    Y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
    eng.op_tile_weight(Wd.data_ptr(), N, K, Wt.data_ptr())
    torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
    eng.op_gemm(Wt.data_ptr(), N, K, Xd.data_ptr(), M, Y.data_ptr())
    eng.sync()
    ref = X.double() @ W.double().t()
    got = Y.cpu().double()
    # one bf16 rounding of the result plus f32 accumulation error (cancellation-aware)
    ulp = torch.maximum(ref.abs(), torch.full_like(ref, 1e-30)).log2().floor().sub(7).exp2()
    acc = (X.double().abs() @ W.double().abs().t()) * (K * 2.0 ** -24)
    excess = (got - ref).abs() - ulp
    assert (excess <= acc).all(), (excess - acc).max().item()
    # row independence: row 0 alone gives the same bits
    Y1 = torch.empty(1, N, dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
    eng.op_gemm(Wt.data_ptr(), N, K, Xd[-1:].contiguous().data_ptr(), 1, Y1.data_ptr())
    eng.sync()
    assert torch.equal(Y1.cpu(), Y[-1:].cpu())


def test_lm_head_argmax(eng, oracle_weights):
    import torch
    E = oracle_weights.p["model.language_model.embed_tokens.weight"]
    g = torch.Generator().manual_seed(5)
    X = torch.randn(5, 1024, generator=g).to(torch.bfloat16)
    X[3] = X[2]
    tok = torch.empty(5, dtype=torch.int32, device="cuda")
    lg = torch.empty(5, 248320, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
    eng.op_lm_head_argmax(X.cuda().data_ptr(), 5, tok.data_ptr(), lg.data_ptr())
    eng.sync()
    lg = lg.cpu()
    ref = (X.float() @ E.float().t())
    # engine logits are bf16 values
    assert torch.equal(lg.to(torch.bfloat16).float(), lg)
    rel = ((lg - ref).abs() / ref.abs().clamp_min(1e-3))
    assert (lg - ref).abs().max().item() < 0.05
    # argmax is the lowest index of the max of the engine's own logits
    for r in range(5):
        row = lg[r]
        m = row.max()
        assert tok[r].item() == int(torch.nonzero(row == m)[0])
    assert tok[2].item() == tok[3].item()


@pytest.mark.parametrize("N,M", [(8224, 600), (5120, 1024), (7168, 768), (1024, 513), (7168, 2048),
                                 (7168, 256), (5120, 256), (8224, 100), (7168, 17), (1024, 300)])
def test_wide_gemm_forms_bit_identical(N, M):
    """The pipelined K = 1024 GEMMs with A in the fragment layout (q35_op_gemm_a amodes 3 / 6:
    256-row blocks at >= 512 rows, 64-row blocks below) equal the batched GEMMs (amodes 0 / 5)
    bit for bit: stored outputs, and the SwiGLU epilogue on [gate; up] weights, including ragged
    last row blocks; the stored form also against float64 (1 bf16 ulp)."""
    mode = 1
    import torch
    from qwen35 import Engine
    print(f"wide gemm mode={mode} N={N} M={M}", flush=True)
    e = Engine(max_rows=2048, max_ctx=64, seed=0)
    try:
        e.set_option("gemm_wide", mode)
        g = torch.Generator().manual_seed(N + M + mode)
        W = (0.02 * torch.randn(N, 1024, generator=g)).to(torch.bfloat16).cuda()
        X = torch.randn(M, 1024, generator=g).to(torch.bfloat16).cuda()
        Wt = torch.empty_like(W)
        ys = [torch.zeros(M, N, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
        ss = [torch.zeros(M, N // 2, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
        torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
        e.op_tile_weight(W.data_ptr(), N, 1024, Wt.data_ptr())
        for am, y in zip((0, 3), ys):
            e.op_gemm_a(Wt.data_ptr(), N, 1024, am, X.data_ptr(), 1024, 0, 0, 0, M, y.data_ptr())
        for am, y in zip((5, 6), ss):
            e.op_gemm_a(Wt.data_ptr(), N, 1024, am, X.data_ptr(), 1024, 0, 0, 0, M, y.data_ptr())
        e.sync()
        assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16))
        assert torch.equal(ss[0].view(torch.int16), ss[1].view(torch.int16))
        ref = X.double() @ W.double().t()
        got = ys[1].double()
        ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
        assert ((got - ref).abs() <= ulp + 1e-6).all()
    finally:
        e.close()
