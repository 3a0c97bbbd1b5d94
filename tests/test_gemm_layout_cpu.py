"""LDS layout maps of the large-problem GEMM kernel (synaptik_amd/csrc/gemm_v2_layout.h), built
for the host: copy placement and fragment addressing are inverse bijections, the kernel's
precomputed fragment offsets match the layout, and fragment reads are free of bank conflicts,
for both tile edges (128 and 64)."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def test_gemm_v2_layout_maps(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "gemm_layout_harness"
    subprocess.run([gxx, "-O1", "-std=c++17", "-o", str(exe), str(HERE / "gemm_layout_harness.cpp")],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.strip()
    assert out == "ok", out
