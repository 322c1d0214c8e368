"""Build ``libbutterfly_amd.so`` (gfx950) in-tree with hipcc.

Usage: ``python -m butterfly_amd.build`` (or ``build()`` from Python).
Always recompiles: the output is what the tests, smoke and bench load.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libbutterfly_amd.so"
SOURCES = ["topology.hip", "compress.hip", "attention.hip", "decode.hip", "streams.hip", "decoder_ops.hip", "qgemv.hip"]
ARCH = os.environ.get("BFLY_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Keep hipcc from forming packed fp32 ops: some of their forms have given
    # silently wrong results on the target boxes.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading pointer arguments of a kernel arrive preloaded in SGPRs (the decode
    # step reads its counters through the first one without a kernel-argument load).
    "-mllvm", "-amdgpu-kernarg-preload-count=2",
    "-Wno-unused-result",
]


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-I", str(PKG.parent / "include"), *[str(CSRC / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
