"""Builds libqwen35.so (all HIP kernels + the C-ABI engine) for gfx950, in-tree.

    python qwen3.5-0.8b_amd/build.py

Each source compiles to an object in qwen3.5-0.8b_amd/_build/ (parallel), then one
`hipcc -shared` link. Packed-FP32 instruction generation is disabled for all device code.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
SRC = PKG / "csrc"
OUT = PKG / "libqwen35.so"
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=off: a * b + c stays two roundings unless a kernel asks for fmaf, so the
# reduction trees and updates written with __fmul_rn / __fadd_rn (plain operators in HIP) round
# the same way in every kernel that shares them
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", str(SRC), "-I", str(PKG.parent / "include")]
# MFMA accumulators in architectural VGPRs: without it the compiler keeps loop-carried
# accumulators in AGPRs and copies them to VGPRs and back around every VALU touch of them
# (the prompt attention's online-softmax rescale: ~190 v_accvgpr moves per K/V tile)
FILE_FLAGS = {"q35_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(SRC.glob("*.hip")) + sorted(SRC.glob("*.cpp"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed\n" + r.stderr)
    os.replace(tmp, OUT)
    if verbose:
        print("built", OUT)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
