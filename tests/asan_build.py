"""Builds an AddressSanitizer variant of libsynaptik_hip.so for host-side tests on the CPU.

The host sources (runtime.cpp, lxm.cpp) are compiled with ASan on their host pass only
(`-Xarch_host -fsanitize=address`; device code cannot be sanitized here) and linked with the
library's already-built kernel objects against the shared ASan runtime. A process loading it must
preload that runtime (LD_PRELOAD), since the Python interpreter itself is not instrumented.
Output: tests/_asan/libsynaptik_hip_asan.so (not part of the product).
"""
from __future__ import annotations

import glob
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
from synaptik_amd import build_native as bn  # noqa: E402

OUT = ROOT / "tests" / "_asan"
LIB = OUT / "libsynaptik_hip_asan.so"
HOST_SOURCES = ["runtime.cpp", "lxm.cpp"]
ASAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]


def asan_runtime() -> str:
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise FileNotFoundError("the clang ASan runtime is not installed")
    return found[-1]


def build() -> Path:
    OUT.mkdir(exist_ok=True)
    objs = []
    for src in bn.SOURCES:
        if src in HOST_SOURCES:
            obj = OUT / (src.replace(".", "_") + ".o")
            cmd = [bn.HIPCC, *bn.COMMON_FLAGS, *ASAN, "-x", "hip", "-c", str(bn.CSRC / src),
                   "-o", str(obj)]
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode:
                raise RuntimeError(res.stderr)
        else:
            obj = bn.OUT_DIR / (src.replace(".", "_") + ".o")
            if not obj.exists():
                bn.build(verbose=False)
        objs.append(obj)
    cmd = [bn.HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Xarch_host",
           "-fsanitize=address", "-shared-libsan", "-o", str(LIB), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(res.stderr)
    return LIB


if __name__ == "__main__":
    print(build())
