"""The binary32 softmax exponential (synaptik_amd/csrc/fexp.h), built for the host with g++ and
compared with the reference addend (float)StrictMath.exp((double)t)
(CpuSoftmaxReferenceKernel.java:104-146; glibc's binary64 exp stands in for StrictMath).

The device kernels compile the same header, so this pins the arithmetic the GPU performs."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("fexp") / "fexp_harness"
    subprocess.run([gxx, "-O2", "-ffp-contract=off", "-o", str(exe), str(HERE / "fexp_harness.cpp"),
                    "-lm"], check=True)
    return exe


def run(exe, stride):
    out = subprocess.run([str(exe), str(stride)], check=True, capture_output=True, text=True)
    n, diff, max_ulp, exact_outside, nan_ok = map(int, out.stdout.split())
    return n, diff, max_ulp, exact_outside, nan_ok


def test_exp_f32_within_one_ulp_of_reference(harness):
    # every 257th binary32 pattern: ~16.7M arguments over all exponents and both signs
    n, diff, max_ulp, exact_outside, nan_ok = run(harness, 257)
    assert n > 16_000_000
    assert max_ulp <= 1
    assert exact_outside == 1  # overflow, subnormal, underflow and infinities take the binary64 path
    assert nan_ok == 1
    # arguments in the fast range are a minority of all patterns; most of them round identically
    assert diff / n < 0.01


def test_exp_f32_dense_softmax_range(harness):
    # a denser pass (every 31st pattern) still stays within one ulp
    n, diff, max_ulp, exact_outside, nan_ok = run(harness, 31)
    assert max_ulp <= 1 and exact_outside == 1 and nan_ok == 1
