"""Torch-CPU restatement of the reference's forward pass (the oracle).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

This follows speccheck/specimpl.py (the reference's "torch CPU path") and
speccheck/mtp.py operation for operation, in the same dtypes and in the same order of
rounding, so that on identical weights it produces the same bits. Each function cites
the lines it restates. It is written for the test suite: one request per `Forward`;
B independent lanes are B instances.

Rounding policy it carries (all of it is the reference's, restated):
  * projections: bf16 x @ bf16 W.T  (torch CPU bf16 GEMM, f32 accumulate, one rounding)
  * zero-centred RMSNorm in f32, affine (1+w), one rounding     (specimpl.py:135-139)
  * GDN conv: 4 taps accumulated in f32, rounded once, bf16 SiLU (specimpl.py:252-268)
  * GDN gates and recurrence in f32                             (specimpl.py:274-294)
  * gated RMSNorm in f32 with one final bf16 rounding           (specimpl.py:142-147,304-305)
  * rope in f32 (table f32), so q/k of attention are f32 after rope (specimpl.py:164-183)
  * attention: f32 scores, f32 softmax, weights rounded to bf16, bf16 P@V (specimpl.py:384-389)
  * MLP: silu and the gate product in bf16                      (specimpl.py:400-407)
  * logits bf16, argmax lowest id on ties                        (specimpl.py:475-476,503)
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .weights import (ATTN_LAYERS, CONV_CH, D_HEAD, D_K, D_MODEL, D_V, GDN_LAYERS, H_V,
                      K_CONV, LM, N_KV, N_LAYERS, N_Q, VOCAB)

EPS = 1e-6
ROPE_THETA = 1e7
ROT_DIM = 64
S_SCALE = D_HEAD ** -0.5            # 1/16
Q_SCALE = D_K ** -0.5
KEY_DIM = H_V * D_K                 # 2048
Q_WIDTH = N_Q * D_HEAD              # 2048
ONLINE_BLK = 64
GDN_CHUNK = 64
EOS_IDS = (248046, 248044)


# ---------------------------------------------------------------- norms
def rmsnorm_zc(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Zero-centred RMSNorm (specimpl.py:135-139)."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)
    return (y * (1.0 + w.float())).to(x.dtype)


def rmsnorm_gated(o: torch.Tensor, z: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Gated RMSNorm with a SiLU(z) gate, plain affine (specimpl.py:142-147)."""
    of = o.float()
    n = (of * torch.rsqrt(of.pow(2).mean(-1, keepdim=True) + EPS)).to(o.dtype)
    n = w * n
    return (n * F.silu(z.float())).to(o.dtype)


# ---------------------------------------------------------------- rope
def rope_cs(positions: torch.Tensor):
    """f32 cos/sin of width 64 for rotary pairs (i, i+32) (specimpl.py:151-156)."""
    i = torch.arange(ROT_DIM // 2, dtype=torch.float32)
    inv = 1.0 / (ROPE_THETA ** (2 * i / ROT_DIM))
    ang = positions.to(torch.float32)[:, None] * inv[None, :]
    return torch.cat([ang.cos(), ang.cos()], -1), torch.cat([ang.sin(), ang.sin()], -1)


def rotate_half(a: torch.Tensor) -> torch.Tensor:
    """(specimpl.py:159-161)"""
    h = a.shape[-1] // 2
    return torch.cat([-a[..., h:], a[..., :h]], -1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate the first 64 dims of each head in f32; the rest pass through. The concat
    promotes the whole head to f32 (specimpl.py:164-183)."""
    rot, rest = x[..., :ROT_DIM], x[..., ROT_DIM:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([rot * c + rotate_half(rot) * s, rest], -1)


# ---------------------------------------------------------------- GDN
def gdn_gates(a_raw, b_raw, A_log, dt_bias):
    """beta = sigmoid(b); g = -exp(A_log) * softplus(a + dt_bias) (specimpl.py:275-277)."""
    beta = torch.sigmoid(b_raw.float())
    g = -A_log.float().exp() * F.softplus(a_raw.float() + dt_bias.float())
    return g, beta


def gdn_conv(raw: torch.Tensor, conv_w: torch.Tensor, win):
    """Causal depthwise conv (kernel 4) over [window ; raw], f32 taps, one rounding,
    bf16 SiLU; returns (u, new window) (specimpl.py:252-268)."""
    T = raw.shape[0]
    C = conv_w.reshape(CONV_CH, K_CONV)
    head = torch.zeros((K_CONV - 1, CONV_CH), dtype=raw.dtype) if win is None else win
    padded = torch.cat([head, raw], 0)
    new_win = padded[-(K_CONV - 1):].clone()
    u = torch.zeros(raw.shape, dtype=torch.float32)
    for j in range(K_CONV):
        u += padded[j:j + T].float() * C[:, j].float()
    return F.silu(u.to(raw.dtype)), new_win


def l2_scale(q: torch.Tensor, k: torch.Tensor):
    """q~ = q/||q|| * 128^-1/2, k~ = k/||k|| in f32 (specimpl.py:281-282)."""
    qn = q.float() * torch.rsqrt(q.float().pow(2).sum(-1, keepdim=True) + 1e-6) * Q_SCALE
    kn = k.float() * torch.rsqrt(k.float().pow(2).sum(-1, keepdim=True) + 1e-6)
    return qn, kn


def gdn_recurrent(qn, kn, v, gam, beta, S):
    """Delta-rule recurrence, token loop (specimpl.py:287-294). S [H,Dk,Dv] f32."""
    T, H = qn.shape[0], qn.shape[1]
    o = torch.zeros((T, H, v.shape[-1]), dtype=torch.float32)
    for t in range(T):
        gam_t, kt, qt, vt, bt = gam[t], kn[t], qn[t], v[t].float(), beta[t]
        S = S * gam_t[:, None, None]
        r = torch.einsum("hkd,hk->hd", S, kt)
        dv = bt[:, None] * (vt - r)
        S = S + torch.einsum("hk,hd->hkd", kt, dv)
        o[t] = torch.einsum("hk,hkd->hd", qt, S)
    return o, S


def gdn_chunk_scan(qn, kn, v, g, beta, S=None, C=GDN_CHUNK):
    """Chunked (UT-transform) form of the same recurrence, chunk 64, right-padded with
    beta = 0 and g = 0 (specimpl.py:187-235)."""
    T, H, DK = kn.shape
    DV = v.shape[-1]
    pad = (-T) % C

    def padseq(x):
        if pad == 0:
            return x
        return torch.cat([x, x.new_zeros((pad,) + tuple(x.shape[1:]))], 0)

    q = padseq(qn).float().transpose(0, 1).reshape(H, -1, C, DK)
    k = padseq(kn).float().transpose(0, 1).reshape(H, -1, C, DK)
    vv = padseq(v).float().transpose(0, 1).reshape(H, -1, C, DV)
    de = padseq(g).float().transpose(0, 1).reshape(H, -1, C)
    be = padseq(beta).float().transpose(0, 1).reshape(H, -1, C)
    NC = q.shape[1]

    v_beta, k_beta = vv * be[..., None], k * be[..., None]
    cum = de.cumsum(-1)
    upper = torch.ones(C, C, dtype=torch.bool).triu(1)
    pair = (cum[..., :, None] - cum[..., None, :]).masked_fill(upper, float("-inf")).exp()
    ut = (k_beta @ k.transpose(-1, -2)) * pair
    intra = (q @ k.transpose(-1, -2)) * pair
    kcd = k_beta * cum.exp()[..., None]
    nv = torch.linalg.solve_triangular(ut, v_beta, upper=False, unitriangular=True)
    kcd = torch.linalg.solve_triangular(ut, kcd, upper=False, unitriangular=True)

    q = q * cum.exp()[..., None]
    k = k * (cum[..., -1:] - cum).exp()[..., None]
    cdec = cum[..., -1].exp()[..., None, None]
    S = torch.zeros((H, DK, DV), dtype=torch.float32) if S is None else S.float()
    out = torch.zeros((H, NC, C, DV), dtype=torch.float32)
    for i in range(NC):
        v_new = nv[:, i] - kcd[:, i] @ S
        out[:, i] = q[:, i] @ S + intra[:, i] @ v_new
        S = S * cdec[:, i] + k[:, i].transpose(-1, -2) @ v_new
    return out.reshape(H, NC * C, DV)[:, :T].transpose(0, 1).contiguous(), S


def gdn_block(w, l: int, x: torch.Tensor, win=None, S=None, form: str = "recurrent",
              dbg: dict | None = None):
    """One GatedDeltaNet mixer over T tokens (specimpl.py:238-310).
    Returns (out [T,1024] bf16, new window [3,6144] bf16, new S [16,128,128] f32)."""
    p = f"{LM}layers.{l}.linear_attn."
    T = x.shape[0]
    raw = x @ w.p[p + "in_proj_qkv.weight"].t()
    z = x @ w.p[p + "in_proj_z.weight"].t()
    b_raw = x @ w.p[p + "in_proj_b.weight"].t()
    a_raw = x @ w.p[p + "in_proj_a.weight"].t()
    u, new_win = gdn_conv(raw, w.p[p + "conv1d.weight"], win)
    q = u[:, :KEY_DIM].reshape(T, H_V, D_K)
    k = u[:, KEY_DIM:2 * KEY_DIM].reshape(T, H_V, D_K)
    v = u[:, 2 * KEY_DIM:].reshape(T, H_V, D_V)
    g, beta = gdn_gates(a_raw, b_raw, w.p[p + "A_log"], w.p[p + "dt_bias"])
    gam = g.exp()
    qn, kn = l2_scale(q, k)
    S = torch.zeros((H_V, D_K, D_V), dtype=torch.float32) if S is None else S
    if form == "chunk" and T > 1:
        o, S = gdn_chunk_scan(qn, kn, v, g, beta, S)
    else:
        o, S = gdn_recurrent(qn, kn, v, gam, beta, S)
    gated = rmsnorm_gated(o.reshape(T * H_V, D_V), z.reshape(T * H_V, D_V),
                          w.p[p + "norm.weight"]).to(raw.dtype)
    if dbg is not None:
        dbg.update(raw=raw, z=z, a=a_raw, b=b_raw, u=u, g=g, beta=beta, o=o, gated=gated,
                   S=S, win=new_win)
    return gated.reshape(T, KEY_DIM) @ w.p[p + "out_proj.weight"].t(), new_win, S


# ---------------------------------------------------------------- attention
def attention_block(w, prefix: str, x: torch.Tensor, cos, sin, kv: dict,
                    softmax: str = "full", dbg: dict | None = None):
    """Gated GQA attention (specimpl.py:320-397). `kv` holds lists "k" (f32 post-rope)
    and "v" (bf16) of [t,2,256] entries; this call appends its T rows."""
    p = prefix
    T = x.shape[0]
    qg = (x @ w.p[p + "q_proj.weight"].t()).view(T, N_Q, D_HEAD * 2)
    q_raw, gate = qg[..., :D_HEAD], qg[..., D_HEAD:]
    k_raw = (x @ w.p[p + "k_proj.weight"].t()).view(T, N_KV, D_HEAD)
    v_raw = (x @ w.p[p + "v_proj.weight"].t()).view(T, N_KV, D_HEAD)
    qh = apply_rope(rmsnorm_zc(q_raw, w.p[p + "q_norm.weight"]), cos, sin)
    kh = apply_rope(rmsnorm_zc(k_raw, w.p[p + "k_norm.weight"]), cos, sin)
    kv.setdefault("k", []).append(kh)
    kv.setdefault("v", []).append(v_raw)
    K = torch.cat(kv["k"], 0)
    V = torch.cat(kv["v"], 0)
    P = K.shape[0]
    out = torch.zeros((T, N_Q, D_HEAD), dtype=x.dtype)
    online = softmax == "online" and T == 1
    for i in range(N_Q):
        j = i // (N_Q // N_KV)
        if online:                                   # specimpl.py:350-372
            srow = ((qh[0, i, :][None, :] @ K[:, j, :].t()) * S_SCALE).float()[0]
            m = torch.full((), float("-inf"), dtype=torch.float32)
            lsum = torch.zeros((), dtype=torch.float32)
            acc = torch.zeros(D_HEAD, dtype=torch.float32)
            for lo in range(0, P, ONLINE_BLK):
                blk = srow[lo:lo + ONLINE_BLK]
                mb = torch.maximum(m, blk.max())
                rescale = torch.exp(m - mb)
                e = torch.exp(blk - mb)
                lsum = lsum * rescale + e.sum()
                acc = acc * rescale + e @ V[lo:lo + ONLINE_BLK, j, :].float()
                m = mb
            out[0, i, :] = (acc / lsum).to(x.dtype)
            continue
        s = (qh[:, i, :] @ K[:, j, :].t()) * S_SCALE          # specimpl.py:384-389
        qi = torch.arange(T)[:, None] + (P - T)
        allowed = torch.arange(P)[None, :] <= qi
        s = s.masked_fill(~allowed, float("-inf"))
        attn = torch.softmax(s.float(), dim=-1).to(x.dtype)
        out[:, i, :] = attn @ V[:, j, :].to(x.dtype)
    pre_gate = out.reshape(T, Q_WIDTH)
    if dbg is not None:
        dbg.update(q_rope=qh, k_rope=kh, v=v_raw, pre_gate=pre_gate, gate=gate)
    gated = pre_gate * torch.sigmoid(gate.reshape(T, Q_WIDTH))
    return gated @ w.p[p + "o_proj.weight"].t()


def mlp_block(w, prefix: str, x: torch.Tensor) -> torch.Tensor:
    """SwiGLU MLP, silu and product in bf16 (specimpl.py:400-407)."""
    gate = x @ w.p[prefix + "gate_proj.weight"].t()
    up = x @ w.p[prefix + "up_proj.weight"].t()
    return (F.silu(gate) * up) @ w.p[prefix + "down_proj.weight"].t()


def argmax_lowest(logits: torch.Tensor) -> int:
    """Greedy id: torch.argmax, which returns the first (lowest) index of the maximum
    (specimpl.py:503, decode_step.cpp:1280-1287 strict '>' scan)."""
    return int(logits.argmax())


# ---------------------------------------------------------------- driver
class Forward:
    """One request's decode state and the 24-layer chain (specimpl.py:410-517)."""

    def __init__(self, w, gdn_form: str = "recurrent", attn_softmax: str = "full"):
        self.w = w
        self.gdn_form = gdn_form
        self.attn_softmax = attn_softmax
        self.generated: list[int] = []
        self.reset()

    def reset(self):
        self.P = 0
        self.kv = {l: {} for l in ATTN_LAYERS}
        self.conv_win = {l: None for l in GDN_LAYERS}
        self.rec = {l: None for l in GDN_LAYERS}

    def _layer(self, l: int, x, cos, sin, form, dbg=None):
        """specimpl.py:426-451"""
        w = self.w
        pre = f"{LM}layers.{l}."
        h = rmsnorm_zc(x, w.p[pre + "input_layernorm.weight"])
        sub = {} if dbg is not None else None
        if l in GDN_LAYERS:
            h, self.conv_win[l], self.rec[l] = gdn_block(
                w, l, h, self.conv_win[l], self.rec[l], form, sub)
        else:
            h = attention_block(w, pre + "self_attn.", h, cos, sin, self.kv[l],
                                self.attn_softmax, sub)
        if dbg is not None:
            dbg[l] = sub
        x = x + h
        h = rmsnorm_zc(x, w.p[pre + "post_attention_layernorm.weight"])
        return x + mlp_block(w, pre + "mlp.", h)

    def _run(self, ids: list[int], form: str, dbg=None):
        x = self.w.p[LM + "embed_tokens.weight"][ids]
        cos, sin = rope_cs(torch.arange(len(ids)) + self.P)
        for l in range(N_LAYERS):
            x = self._layer(l, x, cos, sin, form, dbg)
        self.P += len(ids)
        self.x_final = x
        return rmsnorm_zc(x, self.w.p[LM + "norm.weight"])

    def prefill(self, ids, dbg=None):
        """specimpl.py:457-464"""
        return self._run([int(t) for t in ids], self.gdn_form, dbg)

    def decode(self, tok: int, dbg=None):
        """specimpl.py:466-473"""
        return self._run([int(tok)], "recurrent", dbg)

    def logits(self, normed: torch.Tensor) -> torch.Tensor:
        """Tied lm_head, bf16 (specimpl.py:475-476)."""
        return normed @ self.w.p[LM + "embed_tokens.weight"].t()

    def snapshot(self) -> dict:
        """specimpl.py:478-487"""
        return {"P": self.P, "rec": dict(self.rec), "conv_win": dict(self.conv_win),
                "kv": {l: {n: list(v.get(n, [])) for n in ("k", "v")} for l, v in self.kv.items()}}

    def restore(self, snap: dict):
        """specimpl.py:489-494"""
        self.P = snap["P"]
        self.rec = dict(snap["rec"])
        self.conv_win = dict(snap["conv_win"])
        self.kv = {l: {n: list(v.get(n, [])) for n in ("k", "v")} for l, v in snap["kv"].items()}

    def greedy(self, ids, steps: int, stop_on_eos: bool = True, logits_out=None):
        """specimpl.py:496-517; `logits_out` (a list) receives each step's bf16 logits."""
        out: list[int] = []
        last = self.logits(self.prefill(ids))[-1]
        if logits_out is not None:
            logits_out.append(last)
        out.append(argmax_lowest(last))
        for _ in range(steps):
            if stop_on_eos and out[-1] in EOS_IDS:
                break
            last = self.logits(self.decode(out[-1]))[-1]
            if logits_out is not None:
                logits_out.append(last)
            out.append(argmax_lowest(last))
        self.generated = out
        return out


class MTPDraft:
    """The MTP block as a drafter with its own KV (speccheck/mtp.py:36-83)."""

    def __init__(self, w, softmax: str = "full"):
        self.w = w
        self.softmax = softmax
        self.reset()

    def reset(self):
        self.kv: dict = {}
        self.n = 0

    def snapshot(self):
        return {"k": list(self.kv.get("k", [])), "v": list(self.kv.get("v", []))}

    def restore(self, snap):
        self.kv = {"k": list(snap["k"]), "v": list(snap["v"])}

    def draft(self, y_next: int, h: torch.Tensor, p: int, dbg=None):
        """mtp.py:57-83: e'=RMS(E[y]), h'=RMS(h), u=[e'|h'] W_fc^T, attention at
        position p on the MTP KV, MLP, mtp.norm, tied logits, argmax."""
        w = self.w
        E = w.p[LM + "embed_tokens.weight"]
        e = rmsnorm_zc(E[[y_next]], w.p["mtp.pre_fc_norm_embedding.weight"])
        hh = rmsnorm_zc(h, w.p["mtp.pre_fc_norm_hidden.weight"])
        u = torch.cat([e, hh], -1) @ w.p["mtp.fc.weight"].t()
        pre = "mtp.layers.0."
        cos, sin = rope_cs(torch.tensor([p]))
        z = u + attention_block(w, pre + "self_attn.",
                                rmsnorm_zc(u, w.p[pre + "input_layernorm.weight"]),
                                cos, sin, self.kv, self.softmax)
        z = z + mlp_block(w, pre + "mlp.", rmsnorm_zc(z, w.p[pre + "post_attention_layernorm.weight"]))
        x_d = rmsnorm_zc(z, w.p["mtp.norm.weight"])
        self.n += 1
        logits = (x_d @ E.t())[-1]
        if dbg is not None:
            dbg.update(u=u, x_d=x_d, logits=logits)
        return argmax_lowest(logits), x_d


def greedy_mtp(f: Forward, m: MTPDraft, ids, steps: int, k: int = 1,
               stop_on_eos: bool = True, verify: str = "batch"):
    """Greedy target plus k MTP drafts per target step with greedy accept and rollback
    (speccheck/mtp.py:97-179, post-norm hidden, [emb|hidden] order)."""
    stats = dict(target_forwards=0, drafted=0, accepted=0, bonus=0, verify_tokens=0)

    def feed(seq):
        stats["target_forwards"] += 1
        stats["verify_tokens"] += len(seq)
        if verify == "batch":
            n = f.prefill(seq)
            return n, [argmax_lowest(x) for x in f.logits(n)]
        last, tgt = None, []
        for one in seq:
            last = f.decode(one)
            tgt.append(argmax_lowest(f.logits(last)[-1]))
        return last, tgt

    normed = f.prefill(list(ids))
    stats["target_forwards"] += 1
    t = argmax_lowest(f.logits(normed)[-1])
    out = [t]
    h = normed[-1:]
    while len(out) < steps + 1 and not (stop_on_eos and out[-1] in EOS_IDS):
        q = f.P
        snap, msnap = f.snapshot(), m.snapshot()
        drafts, hd, yd = [], h, t
        for j in range(k):
            d, hd = m.draft(yd, hd, q + 1 + j)
            drafts.append(d)
            yd = d
        stats["drafted"] += k
        normed, tgt = feed([t] + drafts)
        a = 0
        while a < k and drafts[a] == tgt[a]:
            a += 1
        if a < k:
            f.restore(snap)
            m.restore(msnap)
            m.n = len(msnap["k"])
            normed, _ = feed([t] + drafts[:a])
        h = normed[-1:]
        stats["accepted"] += a
        stats["bonus"] += 1
        out.extend(drafts[:a])
        out.append(tgt[a] if a < k else tgt[k])
        t = out[-1]
    f.generated = out
    return out, stats
