"""The benchmark's parity configs on the GPU, op by op through the C ABI.

config 1: every decode projection shape at batch 1, 16 and 256 (W ~ N(0,0.02), x ~ N(0,1)
          bf16), plus the tied lm_head with argmax. Bar: within one bf16 rounding plus the f32
          accumulation bound of the float64 product; rows bit-identical across batch sizes;
          argmax = lowest id of the maximum of the engine's own bf16 logits.
config 2: one GatedDeltaNet decode step at batch 1, 64 and 1024 (inputs N(0,1), state
          N(0,0.1), layer-0 weights) against the oracle's conv / gates / L2 / recurrence
          (speccheck/specimpl.py:252-294). Inputs are identical, so the bar is tight:
          new state max |d| <= 1e-5 + 1e-4 |S|, o max |d| <= 1e-4 max |o|, window exact.
config 3: attention decode at batched lanes over seeded K/V (B 32 / 256, L 1k / 8k) inside
          the full step: logits within the engine-vs-oracle tolerances (max |d| <= 0.375,
          mean |d| <= 0.05), batched lanes bit-identical to the same lane decoded alone.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_MAX, LOGIT_MEAN = 0.375, 0.05

SHAPES = [("in_proj_qkv", 6144, 1024), ("in_proj_z", 2048, 1024), ("in_proj_a", 16, 1024),
          ("out_proj", 1024, 2048), ("q_proj", 4096, 1024), ("k_proj", 512, 1024),
          ("o_proj", 1024, 2048), ("gate_proj", 3584, 1024), ("down_proj", 1024, 3584)]


@pytest.fixture(scope="module")
def eng():
    import torch
    assert torch.cuda.is_available()
    from qwen35 import Engine
    e = Engine(max_rows=256, max_ctx=512, seed=0)
    yield e
    e.close()


@pytest.mark.parametrize("name,N,K", SHAPES)
def test_config1_projection_sweep(eng, name, N, K):
    import torch
    print(f"config1 {name} {K}->{N}", flush=True)
    g = torch.Generator().manual_seed(N * 7 + K)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    X = torch.randn(256, K, generator=g).to(torch.bfloat16)
    Wd = W.cuda()
    Wt = torch.empty_like(Wd)
    torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
    eng.op_tile_weight(Wd.data_ptr(), N, K, Wt.data_ptr())
    outs = {}
    for B in (1, 16, 256):
        Xd = X[:B].contiguous().cuda()
        Y = torch.empty(B, N, dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
        eng.op_gemm(Wt.data_ptr(), N, K, Xd.data_ptr(), B, Y.data_ptr())
        eng.sync()
        outs[B] = Y.cpu()
    ref = X.double() @ W.double().t()
    ulp = torch.maximum(ref.abs(), torch.full_like(ref, 1e-30)).log2().floor().sub(7).exp2()
    acc = (X.double().abs() @ W.double().abs().t()) * (K * 2.0 ** -24)
    got = outs[256].double()
    assert ((got - ref).abs() - ulp <= acc).all()
    assert torch.equal(outs[1], outs[256][:1]) and torch.equal(outs[16], outs[256][:16])


def test_config1_lm_head_argmax(eng, oracle_weights):
    import torch
    E = oracle_weights.p["model.language_model.embed_tokens.weight"]
    g = torch.Generator().manual_seed(11)
    X = torch.randn(256, 1024, generator=g).to(torch.bfloat16)
    res = {}
    for B in (1, 16, 256):
        tok = torch.empty(B, dtype=torch.int32, device="cuda")
        lg = torch.empty(B, 248320, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
        eng.op_lm_head_argmax(X[:B].contiguous().cuda().data_ptr(), B, tok.data_ptr(), lg.data_ptr())
        eng.sync()
        res[B] = (tok.cpu(), lg.cpu())
    tok, lg = res[256]
    assert torch.equal(res[1][1], lg[:1]) and torch.equal(res[16][1], lg[:16])
    for r in range(256):
        row = lg[r]
        assert tok[r].item() == int(torch.nonzero(row == row.max())[0])
    ref = X[:16].double() @ E.double().t()
    assert (lg[:16].double() - ref).abs().max().item() < 0.06


@pytest.mark.parametrize("M", [17, 100, 250, 256])
def test_lm_head_persistent_equals_tiled(eng, M):
    """The persistent lm_head kernels (A resident in LDS with 64 x 32 wave tiles; A in
    registers with the weights streamed through an LDS ring and a running argmax per column
    stream) and the 64 x 256 tiled kernel follow the same reduction order: identical logits and
    tokens, including a ragged last row block (M = 17, 100, 250)."""
    import torch
    print(f"lm_head persistent vs tiled M={M}", flush=True)
    g = torch.Generator().manual_seed(M)
    X = torch.randn(M, 1024, generator=g).to(torch.bfloat16).cuda()
    out = {}
    for p in (0, 1, 3):
        eng.set_option("lmhead_persist", p)
        tok = torch.full((M,), -1, dtype=torch.int32, device="cuda")
        lg = torch.full((M, 248320), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
        eng.op_lm_head_argmax(X.data_ptr(), M, tok.data_ptr(), lg.data_ptr())
        eng.sync()
        out[p] = (tok.cpu(), lg.cpu())
    eng.set_option("lmhead_persist", 3)
    for p in (1, 3):
        assert torch.equal(out[0][0], out[p][0]), p
        assert torch.equal(out[0][1], out[p][1]), p




def test_lm_head_persistent_row_chunks():
    """Above 512 rows (MTP verify at 256 lanes: 768 rows) the persistent lm_head runs in
    launches of 256 rows; tokens and logits equal the tiled kernel's, row offsets included."""
    import torch
    from qwen35 import Engine
    e = Engine(max_rows=768, max_ctx=64, seed=0)
    try:
        M = 700
        X = torch.randn(M, 1024, generator=torch.Generator().manual_seed(700)).to(torch.bfloat16).cuda()
        out = {}
        for p in (0, 1, 3):
            e.set_option("lmhead_persist", p)
            tok = torch.full((M,), -1, dtype=torch.int32, device="cuda")
            lg = torch.full((M, 248320), float("nan"), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
            e.op_lm_head_argmax(X.data_ptr(), M, tok.data_ptr(), lg.data_ptr())
            e.sync()
            out[p] = (tok.cpu(), lg.cpu())
        for p in (1, 3):
            assert torch.equal(out[0][0], out[p][0]), p
            assert torch.equal(out[0][1], out[p][1]), p
    finally:
        e.close()

@pytest.mark.parametrize("N", [1024, 5120, 7168, 8704])
def test_k1024_gemm_forms_identical(eng, N):
    """Batched K = 1024 projections: the all-loads-up-front kernels (32 x 64 blocks and 64 x 128
    blocks of 8 waves, A fragments DMA'd into LDS) and the k-block pipelined kernel give
    identical bits, for ragged (M = 17, 200) and full (M = 256) row counts."""
    import torch
    print(f"k1024 gemm forms N={N}", flush=True)
    g = torch.Generator().manual_seed(N)
    W = (torch.randn(N, 1024, generator=g) * 0.02).to(torch.bfloat16).cuda()
    Wt = torch.empty_like(W)
    torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
    eng.op_tile_weight(W.data_ptr(), N, 1024, Wt.data_ptr())
    for M in (17, 200, 256):
        X = torch.randn(M, 1024, generator=g).to(torch.bfloat16).cuda()
        out = {}
        for p in (0, 1, 2):
            eng.set_option("gemm_pre", p)
            Y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
            torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
            eng.op_gemm(Wt.data_ptr(), N, 1024, X.data_ptr(), M, Y.data_ptr())
            eng.sync()
            out[p] = Y.cpu()
        eng.set_option("gemm_pre", 1)
        assert not torch.isnan(out[0].float()).any()
        assert torch.equal(out[0], out[1]), M
        assert torch.equal(out[0], out[2]), M

@pytest.mark.parametrize("B", [1, 64, 1024])
def test_config2_gdn_step(eng, oracle_weights, B):
    import torch
    from oracle import model
    print(f"config2 gdn B={B}", flush=True)
    p = "model.language_model.layers.0.linear_attn."
    conv_w, A_log, dt_bias = (oracle_weights.p[p + n] for n in ("conv1d.weight", "A_log", "dt_bias"))
    g = torch.Generator().manual_seed(B)
    proj = torch.randn(B, 8224, generator=g).to(torch.bfloat16)
    S0 = (torch.randn(B, 16, 128, 128, generator=g) * 0.1).float()
    W0 = torch.randn(B, 3, 6144, generator=g).to(torch.bfloat16)
    S2 = torch.zeros(B, 2, 16, 128, 128, dtype=torch.float32)
    S2[:, 0] = S0
    W2 = torch.zeros(B, 2, 3, 6144, dtype=torch.float32)
    W2[:, 0] = W0.float()
    dS2, dW2 = S2.cuda(), W2.cuda()
    o = torch.empty(B, 2048, dtype=torch.float32, device="cuda")
    dproj = proj.cuda()
    cw, al, db = conv_w.contiguous().cuda(), A_log.contiguous().cuda(), dt_bias.contiguous().cuda()
    torch.cuda.synchronize()   # torch-stream inputs complete before the engine stream reads them
    eng.op_gdn_step(dproj.data_ptr(), cw.data_ptr(), al.data_ptr(), db.data_ptr(), dS2.data_ptr(),
                    dW2.data_ptr(), o.data_ptr(), B)
    S1, W1, o = dS2[:, 1].cpu(), dW2[:, 1].cpu(), o.cpu()
    lanes = range(B) if B <= 64 else range(0, B, 97)
    for b in lanes:
        raw = proj[b:b + 1, :6144]
        u, win = model.gdn_conv(raw, conv_w, W0[b])
        q = u[:, :2048].reshape(1, 16, 128)
        k = u[:, 2048:4096].reshape(1, 16, 128)
        v = u[:, 4096:].reshape(1, 16, 128)
        gg, beta = model.gdn_gates(proj[b:b + 1, 8208:8224], proj[b:b + 1, 8192:8208], A_log, dt_bias)
        qn, kn = model.l2_scale(q, k)
        ro, rS = model.gdn_recurrent(qn, kn, v, gg.exp(), beta, S0[b].clone())
        assert torch.equal(W1[b], win.float()), b
        dS = (S1[b] - rS).abs()
        assert (dS <= 1e-5 + 1e-4 * rS.abs()).all(), (b, dS.max().item())
        assert (o[b] - ro.reshape(-1)).abs().max().item() <= 1e-4 * ro.abs().max().item() + 1e-7, b


@pytest.mark.parametrize("B,L", [(32, 1024), (256, 1024), (32, 8192), (256, 8192), (32, 32768), (256, 32768)])
def test_config3_attention_batched(oracle_weights, B, L):
    """Benchmark config 3 at batched lanes: B lanes of seeded state (N(0,1) bf16 K/V over L
    slots, N(0,0.1) GDN state) take one decode step (L up to 32,768, config 3's largest). B = 256 at L = 1024 runs the fused
    per-lane attention kernel, the other cases the split slice/part kernels. Checked: lanes 0
    and B-1 against the oracle holding the same state (engine tolerances), and every checked
    lane's logits bit-identical to the same lane decoded alone (single-row path)."""
    from oracle.seeded import seeded_forward
    from qwen35 import Engine, State
    print(f"config3 B={B} L={L}", flush=True)
    e = Engine(max_rows=max(B, 16), max_ctx=L + 64, seed=0)
    toks = [int(t) for t in np.random.default_rng(B + L).integers(0, 248320, B)]
    sb = State(e, B, L + 16)
    sb.seed(1, L)
    out, lg = sb.decode_step(toks, logits=True)
    sb.close()
    s1 = State(e, B, L + 16)
    s1.seed(1, L)
    for lane in (0, B - 1):
        o1, l1 = s1.decode_step([toks[lane]], [lane], logits=True)
        assert np.array_equal(l1[0], lg[lane]), lane
        f = seeded_forward(oracle_weights, 1, lane, L)
        ref = f.logits(f.decode(toks[lane]))[-1].float().numpy()
        d = np.abs(lg[lane] - ref)
        print(f"  lane {lane}: max|d|={d.max():.4f} mean|d|={d.mean():.5f}", flush=True)
        assert d.max() <= LOGIT_MAX and d.mean() <= LOGIT_MEAN
    s1.close()
    e.close()


def test_attention_two_items_per_block_bit_identical():
    """One row per lane at batched lanes runs two (row, kv head) items per attention block
    (engine option attn_pair). With ragged contexts (lanes l and l + 4, which share a block,
    alternate between 300 and 900 cached slots, so the halves run different part counts) and
    100 lanes (the last block has idle halves), logits and tokens equal the one-item blocks'
    bit for bit."""
    from qwen35 import Engine, State
    print("attention two items per block", flush=True)
    B = 100
    e = Engine(max_rows=128, max_ctx=1024, seed=0, use_graph=False)
    try:
        toks = [int(t) for t in np.random.default_rng(5).integers(0, 248320, B)]
        outs = []
        for pair in (1, 0):
            e.set_option("attn_pair", pair)
            short, long_ = State(e, B, 1000), State(e, B, 1000)
            short.seed(3, 300)
            long_.seed(4, 900)
            for ln in range(B):
                if (ln // 4) % 2:
                    long_.copy_lane(ln, short, ln)
            outs.append(short.decode_step(toks, logits=True))
            outs.append(short.decode_step(outs[-1][0], logits=True))
            short.close()
            long_.close()
        for k in range(2):
            assert np.array_equal(outs[k][0], outs[2 + k][0]), k
            assert np.array_equal(outs[k][1].view(np.uint32), outs[2 + k][1].view(np.uint32)), k
    finally:
        e.set_option("attn_pair", 1)
        e.close()


def test_verify_rows_attention_bit_identical():
    """MTP verify bodies at >= 128 lanes run one attention block per (lane, kv head) for the
    lane's 2-3 rows (engine option attn_rows) and their GDN layers in the persistent kernel
    (gdn_rows). With ragged contexts (lanes alternate between 300 and 900 cached slots) and
    128 lanes, a k = 2 round, a k = 1 round and a plain step give the same emits, the same
    final-normed verify rows and the same step logits bit for bit as the one-block-per-row
    attention kernel and the one-block-per-(lane, head) GDN kernel."""
    from qwen35 import Engine, State
    print("verify rows attention", flush=True)
    B = 128
    e = Engine(max_rows=3 * B, max_ctx=1024, seed=0, use_graph=False)
    try:
        toks = [int(t) for t in np.random.default_rng(6).integers(0, 248320, B)]
        outs = []
        for rows in (2, 1, 0):       # 8-wave and 4-wave rows blocks, then one block per row
            e.set_option("attn_rows", rows)
            e.set_option("gdn_rows", min(rows, 1))
            short, long_ = State(e, B, 1000, mtp_k=2, mtp_cap=64), State(e, B, 1000, mtp_k=2, mtp_cap=64)
            short.seed(3, 300)
            long_.seed(4, 900)
            for ln in range(B):
                if ln % 2:
                    long_.copy_lane(ln, short, ln)
            long_.close()
            res = []
            em = short.mtp_round(toks, 2)
            res.append(em)
            res.append(e.read_scratch("nrm", (3 * B, 1024), np.uint16))
            em1 = short.mtp_round([x[-1] for x in em], 1)
            res.append(em1)
            res.append(e.read_scratch("nrm", (2 * B, 1024), np.uint16))
            res.append(short.decode_step([x[-1] for x in em1], logits=True))
            short.close()
            outs.append(res)
        b = outs[-1]
        for a in outs[:-1]:
            assert a[0] == b[0] and a[2] == b[2]
            assert np.array_equal(a[1], b[1]) and np.array_equal(a[3], b[3])
            assert np.array_equal(a[4][0], b[4][0])
            assert np.array_equal(a[4][1].view(np.uint32), b[4][1].view(np.uint32))
    finally:
        e.set_option("attn_rows", 2)
        e.set_option("gdn_rows", 1)
        e.close()
