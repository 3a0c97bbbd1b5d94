"""The public headers are plain C: a C99 translation unit that includes both and takes the address
of every declared entry point compiles warning-free under -pedantic, links against
libsynaptik_hip.so and runs (the device-free calls only), as a binding generated from the
headers (jextract for the FFM binding, cgo, a ctypes stub) would see them."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from synaptik_amd import native

ROOT = Path(__file__).resolve().parent.parent
INCLUDE = ROOT / "include"
ROCM_LIB = Path("/opt/rocm/lib")


def _declared(header: str) -> list[str]:
    text = (INCLUDE / header).read_text()
    return sorted(set(re.findall(r"\b(shk_[a-z0-9_]+)\s*\(", text)))


def _program(names: list[str]) -> str:
    table = ",\n".join(f"    (fn)&{n}" for n in names)
    return f"""#include <stdio.h>
#include <string.h>
#include "synaptik_hip.h"
#include "synaptik_init.h"

typedef void (*fn)(void);
static const fn entry_points[] = {{
{table}
}};

int main(void) {{
    uint64_t state[4];
    int64_t draws[2];
    char msg[64];
    size_t i;
    for (i = 0; i < sizeof entry_points / sizeof entry_points[0]; ++i)
        if (entry_points[i] == NULL) return 10;
    if (shk_hip_abi_version() != SHK_HIP_ABI_VERSION) return 11;
    if (shk_hip_context_create(0, NULL) != SHK_HIP_STATUS_INVALID_ARGUMENT) return 12;
    if (shk_hip_last_error(msg, sizeof msg) != SHK_HIP_STATUS_OK || strlen(msg) == 0) return 13;
    if (shk_lxm_seed(42, state) != 0 || shk_lxm_next_long(state, 2, draws) != 0) return 14;
    printf("%u %lld %lld\\n", (unsigned)shk_hip_abi_version(), (long long)draws[0],
           (long long)draws[1]);
    return 0;
}}
"""


@pytest.fixture(scope="module")
def gcc():
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("no C compiler")
    if not native.LIBRARY_PATH.exists():
        pytest.skip("libsynaptik_hip.so not built (run __graft_entry__.build())")
    return cc


def test_headers_compile_as_pedantic_c99(gcc, tmp_path):
    names = _declared("synaptik_hip.h") + _declared("synaptik_init.h")
    assert _declared("synaptik_hip.h") == sorted(native.EXPORTED_SYMBOLS)
    src = tmp_path / "abi.c"
    src.write_text(_program(names))
    r = subprocess.run([gcc, "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-c",
                        "-I", str(INCLUDE), str(src), "-o", str(tmp_path / "abi.o")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_c_program_links_and_runs_device_free_calls(gcc, tmp_path):
    names = _declared("synaptik_hip.h") + _declared("synaptik_init.h")
    src = tmp_path / "abi.c"
    src.write_text(_program(names))
    exe = tmp_path / "abi"
    libdir = native.LIBRARY_PATH.parent
    r = subprocess.run([gcc, "-std=c99", "-I", str(INCLUDE), str(src), "-o", str(exe),
                        "-L", str(libdir), "-lsynaptik_hip", f"-Wl,-rpath,{libdir}",
                        f"-Wl,-rpath-link,{ROCM_LIB}", f"-Wl,-rpath,{ROCM_LIB}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, (run.returncode, run.stderr)
    version, a, b = run.stdout.split()
    assert int(version) == native.ABI_VERSION
    # the same draws through the Python binding of the same library
    from synaptik_amd.initializers import L64X128MixRandom
    g = L64X128MixRandom(42)
    assert [int(a), int(b)] == [g.next_long(), g.next_long()]
