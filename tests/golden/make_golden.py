"""Writes tests/golden/*.npz from the reference's own torch-CPU path.

Run in the build container only (it imports /root/reference/speccheck/specimpl.py and
speccheck/mtp.py, which never travel to the GPU box):

    python tests/golden/make_golden.py

Inputs are this build's synthetic weights (oracle/weights.py, seed 0) injected into
specimpl's `Weights` without reading a checkpoint. Outputs are data only: token ids,
sha256 digests of full bf16 logits rows / states, top-k logits, small tensors.
"""
from __future__ import annotations

import hashlib
import sys
import time
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
sys.path.insert(0, "/root/reference")

from oracle.weights import WeightDict, prompt_ids  # noqa: E402
from speccheck import specimpl, mtp  # noqa: E402

OUT = Path(__file__).resolve().parent


def digest(t: torch.Tensor) -> str:
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        b = t.view(torch.int16).numpy().tobytes()
    else:
        b = t.numpy().tobytes()
    return hashlib.sha256(b).hexdigest()


def topk_bits(row: torch.Tensor, k: int = 32):
    v, i = torch.topk(row.float(), k)
    return i.numpy().astype(np.int32), v.numpy().astype(np.float32)


def main():
    torch.set_grad_enabled(False)
    t0 = time.time()
    mine = WeightDict(0)
    w = object.__new__(specimpl.Weights)
    w.p = mine.p
    w.dtype = torch.bfloat16
    ids = prompt_ids(0, 32)
    print("weights", time.time() - t0)

    # config 0: prompt of 32 ids, greedy 64 tokens, no EOS stop
    f = specimpl.Forward(w)
    dbg_p, dbg_d = {}, {}
    gen = f.greedy(ids, 64, dbg_p, dbg_d, stop_on_eos=False)
    print("greedy", time.time() - t0, gen[:8])
    rows = [dbg_p["logits_last"][0]] + [dbg_d[f"decode{s}"]["logits_last"] for s in range(64)]
    top_i = np.stack([topk_bits(r)[0] for r in rows])
    top_v = np.stack([topk_bits(r)[1] for r in rows])
    logit_digest = np.array([digest(r) for r in rows])
    layer_keys = sorted(k for k in dbg_p if k.endswith(".s_out"))
    prefill_layer_digest = np.array([digest(dbg_p[k]) for k in layer_keys])
    gdn_state_digest = np.array([digest(f.rec[l]) for l in specimpl.GDN_LAYERS])
    np.savez_compressed(
        OUT / "config0_greedy.npz", prompt=np.array(ids, np.int32), tokens=np.array(gen, np.int32),
        top_i=top_i, top_v=top_v, logit_digest=logit_digest,
        prefill_layer_digest=prefill_layer_digest, final_gdn_state_digest=gdn_state_digest,
        logits0=rows[0].float().numpy()[:4096], logits64=rows[64].float().numpy()[:4096],
        s_out_L00=dbg_p["L00.s_out"].float().numpy(), s_out_L03=dbg_p["L03.s_out"].float().numpy())

    # chunked prefill form (S04.7) of the same prompt
    fc = specimpl.Forward(w, gdn_form="chunk")
    n = fc.prefill(torch.tensor(ids))
    lc = fc.logits(n)[-1]
    np.savez_compressed(
        OUT / "config0_chunk_prefill.npz", logit_digest=np.array([digest(lc)]),
        top_i=topk_bits(lc)[0], top_v=topk_bits(lc)[1],
        gdn_state_digest=np.array([digest(fc.rec[l]) for l in specimpl.GDN_LAYERS]),
        state_L00=fc.rec[0].numpy()[:2])
    print("chunk", time.time() - t0)

    # online softmax decode (S07.3), 8 steps
    fo = specimpl.Forward(w, attn_softmax="online")
    geno = fo.greedy(ids, 8, stop_on_eos=False)
    np.savez_compressed(OUT / "config0_online.npz", tokens=np.array(geno, np.int32))

    # MTP k=2, batched verify and sequential verify, 16 steps
    res = {}
    for verify in ("batch", "steps"):
        f2 = specimpl.Forward(w)
        m = mtp.MTPDraft(w, h_source="post_norm", fc_order="eh")
        out, st = mtp.greedy_mtp(f2, m, ids, 16, k=2, stop_on_eos=False, verify=verify)
        res[verify] = (out, st, f2.P, len(m.kv.get("k", [])))
        print("mtp", verify, time.time() - t0, st)
    # one draft from the prompt's state, for the draft-layer parity
    f3 = specimpl.Forward(w)
    normed = f3.prefill(torch.tensor(ids))
    t = int(f3.logits(normed)[-1].argmax())
    m3 = mtp.MTPDraft(w, h_source="post_norm", fc_order="eh")
    dd = {}
    d1, xd = m3.draft(t, normed[-1:], f3.P + 1, dd)
    np.savez_compressed(
        OUT / "mtp_k2.npz",
        batch_tokens=np.array(res["batch"][0], np.int32),
        batch_stats=np.array([res["batch"][1][k] for k in ("target_forwards", "drafted", "accepted", "bonus", "verify_tokens")]),
        batch_P=np.array(res["batch"][2]), batch_mtp_len=np.array(res["batch"][3]),
        steps_tokens=np.array(res["steps"][0], np.int32),
        steps_stats=np.array([res["steps"][1][k] for k in ("target_forwards", "drafted", "accepted", "bonus", "verify_tokens")]),
        steps_P=np.array(res["steps"][2]), steps_mtp_len=np.array(res["steps"][3]),
        draft1=np.array(d1), draft1_xd=xd.float().numpy(), draft1_logit_digest=np.array([digest(dd["mtp.logits_last"][-1])]),
        draft1_top_i=topk_bits(dd["mtp.logits_last"][-1])[0], draft1_top_v=topk_bits(dd["mtp.logits_last"][-1])[1])
    print("done", time.time() - t0)


if __name__ == "__main__":
    main()
