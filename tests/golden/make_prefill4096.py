"""Writes tests/golden/prefill4096.npz: the oracle's chunked prefill (the reference's chunk
form, speccheck/specimpl.py:187-235 with gdn_form="chunk", restated in oracle/model.py and
pinned bit-exact to the reference's own vectors in the build container's CPU suite) of one
4,096-token prompt: benchmark config 2's T = 4096 case.

    python tests/golden/make_prefill4096.py

Run in the build container (CPU, a few minutes). Outputs are data only: the prompt ids, every
row's greedy id and top-1 / top-2 logit values, the last row's top-32 and first 4,096 logits,
and per GDN layer a strided sample S[:, ::8, ::8] of the final state plus its Frobenius norm.
"""
from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))

from oracle import model  # noqa: E402
from oracle.weights import WeightDict, lane_prompt_ids  # noqa: E402

OUT = Path(__file__).resolve().parent / "prefill4096.npz"
N = 4096


def main():
    torch.set_grad_enabled(False)
    t0 = time.time()
    w = WeightDict(0)
    ids = lane_prompt_ids(4096, 0, N)
    f = model.Forward(w, gdn_form="chunk")
    normed = f.prefill(ids)
    print("prefill", round(time.time() - t0, 1), flush=True)
    E = w.p[model.LM + "embed_tokens.weight"]
    am = np.empty(N, np.int32)
    t1 = np.empty(N, np.float32)
    t2 = np.empty(N, np.float32)
    for r0 in range(0, N, 128):
        lg = (normed[r0:r0 + 128] @ E.t()).float()
        am[r0:r0 + 128] = lg.argmax(-1).numpy()
        v = torch.topk(lg, 2, dim=-1).values.numpy()
        t1[r0:r0 + 128], t2[r0:r0 + 128] = v[:, 0], v[:, 1]
    last = (normed[-1:] @ E.t())[0].float()
    v, i = torch.topk(last, 32)
    print("logits", round(time.time() - t0, 1), flush=True)
    S = np.stack([f.rec[l].numpy()[:, ::8, ::8] for l in model.GDN_LAYERS])
    Sn = np.array([float(np.linalg.norm(f.rec[l].numpy())) for l in model.GDN_LAYERS], np.float64)
    np.savez_compressed(OUT, ids=np.array(ids, np.int32), argmax=am, top1=t1, top2=t2,
                        last_top_i=i.numpy().astype(np.int32), last_top_v=v.numpy().astype(np.float32),
                        last_logits=last.numpy()[:4096], S_sample=S.astype(np.float32), S_norm=Sn)
    print("done", round(time.time() - t0, 1), OUT, flush=True)


if __name__ == "__main__":
    main()
