"""float64 brute-force forms of the decode-path math, used to pin oracle/model.py.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Written from the mathematics in
specification/03-05 (RMSNorm, gated RMSNorm, partial rope, delta-rule recurrence, softmax
attention), independently of model.py's torch code: plain loops / numpy in float64.
"""
from __future__ import annotations

import numpy as np

EPS = 1e-6


def rmsnorm_zc(x, w):
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + EPS) * (1.0 + np.asarray(w, np.float64))


def rmsnorm_gated(o, z, w):
    o = np.asarray(o, np.float64)
    z = np.asarray(z, np.float64)
    n = o / np.sqrt((o * o).mean(-1, keepdims=True) + EPS)
    return np.asarray(w, np.float64) * n * (z / (1.0 + np.exp(-z)))


def rope(x, pos, theta=1e7, rot=64):
    """Rotate pairs (i, i + rot/2) of the first `rot` dims by pos * theta^(-2i/rot)."""
    x = np.array(x, np.float64)
    out = x.copy()
    h = rot // 2
    for i in range(h):
        ang = pos * theta ** (-2.0 * i / rot)
        c, s = np.cos(ang), np.sin(ang)
        a, b = x[..., i], x[..., i + h]
        out[..., i] = a * c - b * s
        out[..., i + h] = b * c + a * s
    return out


def causal_conv(raw, C, win):
    """u[t, c] = sum_j padded[t + j, c] * C[c, j] over [win (3 rows); raw]."""
    padded = np.concatenate([np.asarray(win, np.float64), np.asarray(raw, np.float64)], 0)
    T = raw.shape[0]
    u = np.zeros(raw.shape)
    for t in range(T):
        for j in range(4):
            u[t] += padded[t + j] * C[:, j]
    return u, padded[-3:]


def gates(a, b, A_log, dt_bias):
    x = np.asarray(a, np.float64) + dt_bias
    sp = np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))
    return -np.exp(A_log) * sp, 1.0 / (1.0 + np.exp(-np.asarray(b, np.float64)))


def delta_rule(qn, kn, v, g, beta, S):
    """Token loop of S <- e^g S; S += k (beta (v - S^T k))^T; o = S^T q, per head."""
    S = np.array(S, np.float64)
    T, H, _ = qn.shape
    o = np.zeros((T, H, v.shape[-1]))
    for t in range(T):
        for h in range(H):
            S[h] *= np.exp(g[t, h])
            r = S[h].T @ kn[t, h]
            S[h] += np.outer(kn[t, h], beta[t, h] * (v[t, h] - r))
            o[t, h] = S[h].T @ qn[t, h]
    return o, S


def attention_row(q, K, V, scale=1.0 / 16):
    s = (K @ q) * scale
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ V
