"""The host shim under AddressSanitizer (tests/asan_build.py): a child process with the ASan
runtime preloaded runs tests/asan_driver.py against the sanitized library; it must finish cleanly
with no sanitizer report."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def test_host_shim_is_clean_under_address_sanitizer():
    from tests import asan_build
    try:
        runtime = asan_build.asan_runtime()
    except FileNotFoundError as e:
        pytest.skip(str(e))
    lib = asan_build.build()
    env = dict(os.environ, LD_PRELOAD=runtime,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0:exitcode=99",
               PYTHONPATH=str(HERE.parent))
    res = subprocess.run([sys.executable, str(HERE / "asan_driver.py"), str(lib)], env=env,
                         capture_output=True, text=True, timeout=600)
    assert "AddressSanitizer" not in res.stderr, res.stderr[-4000:]
    assert res.returncode == 0, res.stderr[-4000:]
    assert "asan driver ok" in res.stdout
