"""Tensor registry and the synthetic weight dict (config 0 init).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Names and shapes follow speccheck/specimpl.py:92-127 (the G1 shape table) and
speccheck/mtp.py:64-77 / specification/01-weights-and-shapes.md:71-84 for `mtp.*`.
Every tensor is loaded as bf16, as specimpl's `Weights(dtype=torch.bfloat16)` does by
default (specimpl.py:70-85, keep_f32_scalars=False).

Init (benchmark config 0): matrices, embedding and conv N(0,0.02); RMSNorm weights and
the gated-norm weight 1.0; A_log = log U(1,16); dt_bias ~ U(-1,1). Stream ids are
fnv1a64(name); see prng.c for the stream definition.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import prng

D_MODEL, N_LAYERS, D_FF, VOCAB = 1024, 24, 3584, 248320
N_Q, N_KV, D_HEAD = 8, 2, 256
H_V, D_K, D_V, K_CONV = 16, 128, 128, 4
CONV_CH = 6144
GDN_LAYERS = [i for i in range(N_LAYERS) if (i + 1) % 4 != 0]
ATTN_LAYERS = [i for i in range(N_LAYERS) if (i + 1) % 4 == 0]
STD = 0.02
LM = "model.language_model."


def registry() -> list[tuple[str, tuple[int, ...], str]]:
    """(name, shape, init kind) for every text-tower + MTP tensor, in a fixed order."""
    out: list[tuple[str, tuple[int, ...], str]] = []
    for l in range(N_LAYERS):
        pre = f"{LM}layers.{l}."
        out.append((pre + "input_layernorm.weight", (D_MODEL,), "one"))
        out.append((pre + "post_attention_layernorm.weight", (D_MODEL,), "one"))
        if l in GDN_LAYERS:
            la = pre + "linear_attn."
            out += [(la + "in_proj_qkv.weight", (CONV_CH, D_MODEL), "normal"),
                    (la + "in_proj_z.weight", (2048, D_MODEL), "normal"),
                    (la + "in_proj_b.weight", (H_V, D_MODEL), "normal"),
                    (la + "in_proj_a.weight", (H_V, D_MODEL), "normal"),
                    (la + "conv1d.weight", (CONV_CH, 1, K_CONV), "normal"),
                    (la + "A_log", (H_V,), "alog"),
                    (la + "dt_bias", (H_V,), "dtbias"),
                    (la + "norm.weight", (D_V,), "one"),
                    (la + "out_proj.weight", (D_MODEL, 2048), "normal")]
        else:
            out += _attn(pre + "self_attn.")
        out += _mlp(pre + "mlp.")
    out.append((LM + "embed_tokens.weight", (VOCAB, D_MODEL), "normal"))
    out.append((LM + "norm.weight", (D_MODEL,), "one"))
    out.append(("mtp.pre_fc_norm_embedding.weight", (D_MODEL,), "one"))
    out.append(("mtp.pre_fc_norm_hidden.weight", (D_MODEL,), "one"))
    out.append(("mtp.fc.weight", (D_MODEL, 2 * D_MODEL), "normal"))
    out.append(("mtp.layers.0.input_layernorm.weight", (D_MODEL,), "one"))
    out += _attn("mtp.layers.0.self_attn.")
    out.append(("mtp.layers.0.post_attention_layernorm.weight", (D_MODEL,), "one"))
    out += _mlp("mtp.layers.0.mlp.")
    out.append(("mtp.norm.weight", (D_MODEL,), "one"))
    return out


def _attn(p: str):
    return [(p + "q_proj.weight", (2 * N_Q * D_HEAD, D_MODEL), "normal"),
            (p + "k_proj.weight", (N_KV * D_HEAD, D_MODEL), "normal"),
            (p + "v_proj.weight", (N_KV * D_HEAD, D_MODEL), "normal"),
            (p + "q_norm.weight", (D_HEAD,), "one"),
            (p + "k_norm.weight", (D_HEAD,), "one"),
            (p + "o_proj.weight", (D_MODEL, N_Q * D_HEAD), "normal")]


def _mlp(p: str):
    return [(p + "gate_proj.weight", (D_FF, D_MODEL), "normal"),
            (p + "up_proj.weight", (D_FF, D_MODEL), "normal"),
            (p + "down_proj.weight", (D_MODEL, D_FF), "normal")]


def tensor_bits(seed: int, name: str, shape, kind: str) -> np.ndarray:
    """bf16 bits (uint16) of one tensor, flattened in row-major order."""
    n = int(np.prod(shape))
    tid = prng.fnv1a64(name)
    if kind == "normal":
        return prng.normal_bf16(seed, tid, STD, n)
    if kind == "one":
        return np.full(n, 0x3F80, dtype=np.uint16)
    u = prng.uniform(seed, tid, n).astype(np.float64)
    if kind == "alog":
        v = np.log(1.0 + 15.0 * u)
    elif kind == "dtbias":
        v = -1.0 + 2.0 * u
    else:
        raise ValueError(kind)
    return prng.f32_to_bf16_bits(v.astype(np.float32))


def bits_to_bf16(bits: np.ndarray, shape) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16).reshape(shape)


class WeightDict:
    """Duck-types specimpl.Weights: `.p` maps the checkpoint names to bf16 tensors."""

    def __init__(self, seed: int = 0):
        self.seed = seed
        self.p: dict[str, torch.Tensor] = {}
        for name, shape, kind in registry():
            self.p[name] = bits_to_bf16(tensor_bits(seed, name, shape, kind), shape)


def prompt_ids(seed: int = 0, n: int = 32) -> list[int]:
    """Config 0 prompt: n ids uniform in [0, VOCAB)."""
    return [int(t) for t in prng.tokens(seed, prng.fnv1a64("input.prompt_ids"), n, VOCAB)]


def lane_prompt_ids(seed: int, lane: int, n: int) -> list[int]:
    return [int(t) for t in prng.tokens(seed, prng.fnv1a64(f"input.lane{lane}.prompt_ids"), n, VOCAB)]


def checksum(bits: np.ndarray) -> int:
    """Order-sensitive 64-bit checksum of a uint16 array (FNV-1a over 64-bit words of
    4 elements, tail zero-padded); the device generator's test compares these."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    pad = (-len(b)) % 4
    if pad:
        b = np.concatenate([b, np.zeros(pad, np.uint16)])
    w = b.view(np.uint64)
    # position-weighted sum modulo 2^64: cheap, order-sensitive, vectorised
    with np.errstate(over="ignore"):
        idx = np.arange(1, len(w) + 1, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)
        return int(np.sum(w ^ idx, dtype=np.uint64))
