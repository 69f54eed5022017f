"""Oracle-side restatement of the engine's seeded benchmark state (q35_state_seed).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Lane `lane` of a state seeded with
`seed` at prefix length P holds: GDN S ~ N(0, 0.1) f32 from stream "state.gdn.<lane>",
conv window zero, and K / V ~ N(0, 1) bf16 from streams "state.k.<lane>.<a>.<j>" /
"state.v.<lane>.<a>.<j>" for attention layer a and kv head j, slots [0, P).
"""
from __future__ import annotations

import numpy as np
import torch

from . import model, prng
from .weights import ATTN_LAYERS, GDN_LAYERS


def seeded_forward(w, seed: int, lane: int, P: int) -> model.Forward:
    f = model.Forward(w)
    S_all = prng.normal_f32(seed, prng.fnv1a64(f"state.gdn.{lane}"), 0.1, 18 * 262144).reshape(18, 16, 128, 128)
    for i, l in enumerate(GDN_LAYERS):
        f.rec[l] = torch.from_numpy(S_all[i].copy())
        f.conv_win[l] = torch.zeros(3, 6144, dtype=torch.bfloat16)
    for a, l in enumerate(ATTN_LAYERS):
        ks, vs = [], []
        for j in range(2):
            tag = f"{lane}.{a}.{j}"
            kb = prng.normal_bf16(seed, prng.fnv1a64("state.k." + tag), 1.0, P * 256)
            vb = prng.normal_bf16(seed, prng.fnv1a64("state.v." + tag), 1.0, P * 256)
            ks.append(torch.from_numpy((kb.astype(np.uint32) << 16).view(np.float32).reshape(P, 256)))
            vs.append(torch.from_numpy(vb.view(np.int16).copy()).view(torch.bfloat16).reshape(P, 256))
        f.kv[l] = {"k": [torch.stack(ks, 1)], "v": [torch.stack(vs, 1)]}
    f.P = P
    return f
