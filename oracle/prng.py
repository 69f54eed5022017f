"""Portable seeded generator (numpy restatement + ctypes binding of prng.c).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). The stream definition is in
oracle/prng.c's header; `normal_bf16_np` restates it in numpy so the C build is
itself checked on small slices.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None
M64 = (1 << 64) - 1


def fnv1a64(name: str) -> int:
    """Stream id of a named tensor: FNV-1a 64 over its UTF-8 bytes."""
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & M64
    return h


def _mix_np(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def _mix(x: int) -> int:
    z = (x + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def key(seed: int, tid: int) -> int:
    return _mix((_mix(seed) + tid) & M64)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (NaN kept quiet)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7F800000) == 0x7F800000
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def normal_f32_np(seed: int, tid: int, std: float, start: int, n: int) -> np.ndarray:
    k = np.uint64(key(seed, tid))
    i = np.arange(start, start + n, dtype=np.uint64)
    s = np.zeros(n, dtype=np.int64)
    for j in range(3):
        with np.errstate(over="ignore"):
            r = _mix_np(k + np.uint64(3) * i + np.uint64(j))
        for sh in (0, 16, 32, 48):
            s += ((r >> np.uint64(sh)) & np.uint64(0xFFFF)).astype(np.int64)
    z = (s - 393210).astype(np.float32)
    return z * np.float32(std / 65536.0)


def normal_bf16_np(seed: int, tid: int, std: float, start: int, n: int) -> np.ndarray:
    return f32_to_bf16_bits(normal_f32_np(seed, tid, std, start, n))


def uniform_np(seed: int, tid: int, start: int, n: int) -> np.ndarray:
    k = np.uint64(key(seed, tid))
    i = np.arange(start, start + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        r = _mix_np(k + np.uint64(3) * i)
    return (r >> np.uint64(40)).astype(np.float32) * np.float32(1.0 / 16777216.0)


def tokens_np(seed: int, tid: int, n: int, vocab: int) -> np.ndarray:
    k = np.uint64(key(seed, tid))
    i = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        r = _mix_np(k + np.uint64(3) * i)
    return ((r >> np.uint64(32)) % np.uint64(vocab)).astype(np.int32)


def lib():
    """The C build of the same stream (fast path for the 760 M weight elements)."""
    global _LIB
    if _LIB is None:
        so = _HERE / "liboracle_prng.so"
        if not so.exists() or so.stat().st_mtime < (_HERE / "prng.c").stat().st_mtime:
            subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
        L = ctypes.CDLL(str(so))
        u64, f32, p = ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p
        L.q35o_normal_bf16.argtypes = [u64, u64, f32, u64, u64, p]
        L.q35o_normal_f32.argtypes = [u64, u64, f32, u64, u64, p]
        L.q35o_uniform_f32.argtypes = [u64, u64, u64, u64, p]
        L.q35o_tokens.argtypes = [u64, u64, u64, ctypes.c_uint32, p]
        _LIB = L
    return _LIB


def normal_bf16(seed: int, tid: int, std: float, n: int, start: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().q35o_normal_bf16(seed, tid, std, start, n, out.ctypes.data)
    return out


def normal_f32(seed: int, tid: int, std: float, n: int, start: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().q35o_normal_f32(seed, tid, std, start, n, out.ctypes.data)
    return out


def uniform(seed: int, tid: int, n: int, start: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().q35o_uniform_f32(seed, tid, start, n, out.ctypes.data)
    return out


def tokens(seed: int, tid: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().q35o_tokens(seed, tid, n, vocab, out.ctypes.data)
    return out
