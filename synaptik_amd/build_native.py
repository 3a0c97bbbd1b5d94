"""Builds libsynaptik_hip.so (gfx950) in-tree with hipcc.

Every HIP source is compiled for gfx950 only, with -ffp-contract=off (elementwise kernels
perform exactly the rounded operations the oracle performs) and with packed-fp32 VALU
instructions disabled. Objects go to synaptik_amd/_build/, the shared library to
synaptik_amd/libsynaptik_hip.so, which the GPU box receives with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIBRARY = PKG / "libsynaptik_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# the per-layout GEMM units are the slowest to compile and go first
SOURCES = ["gemm_nn.hip", "gemm_nt.hip", "gemm_tn.hip", "gemm_tt.hip", "gemm.hip", "gemm_skinny.hip",
           "elementwise.hip", "softmax_loss.hip", "ce_head.hip", "optim.hip", "publish.hip", "runtime.cpp", "lxm.cpp"]

COMMON_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _compile(src: str) -> Path:
    obj = OUT_DIR / (src.replace(".", "_") + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    OUT_DIR.mkdir(exist_ok=True)
    workers = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build()
