"""Exercises the device-free entry points of the ASan build of libsynaptik_hip.so: the program
image decoder (valid images of every lowering, then truncations, bit flips and hostile field
values), storage-transfer geometry checks, the LXM generator, and null / foreign handles on every
entry point that checks them before touching a device. Run by tests/test_asan_cpu.py in a child
process with the ASan runtime preloaded; any sanitizer report aborts it."""
import ctypes
import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from synaptik_amd import native  # noqa: E402

lib = native.load_library(sys.argv[1])
from synaptik_amd import program as P  # noqa: E402
from synaptik_amd.backend import HipPartitionPreparer  # noqa: E402
from synaptik_amd.initializers import L64X128MixRandom  # noqa: E402
from synaptik_amd.training import (Adam, GradientMode, MlpSpec, Sgd, lower_dense_layer,  # noqa: E402
                                   lower_forward, lower_training_step)
from tests.partitions import mlp_train_partition, softmax_ce_partition  # noqa: E402


def images():
    out = []
    for spec, opt in ((MlpSpec.chain([16, 64, 1], hidden="tanh"), Sgd(0.01)),
                      (MlpSpec.chain([784, 128, 10], hidden="relu", loss="ce"), Adam(1e-3)),
                      (MlpSpec.chain([32, 32, 32, 8], hidden="sigmoid"), Sgd(0.1, momentum=0.9))):
        for mode in (GradientMode.RESET_AND_STEP, GradientMode.ACCUMULATE,
                     GradientMode.ACCUMULATE_AND_STEP):
            pb, _ = lower_training_step(spec, 64, opt, mode=mode)
            out.append(pb.image())
        out.append(lower_forward(spec, 7).image())
    out.append(lower_dense_layer(64, 32, 48, "relu")[0].image())
    for part in (mlp_train_partition(16, 8, 12, 4), softmax_ce_partition(30, 10)):
        out.append(HipPartitionPreparer().analyze(part).plan)
    return out


def validate(img: bytes) -> int:
    buf = ctypes.create_string_buffer(img, max(1, len(img)))
    arena = ctypes.c_uint64()
    st = lib.shk_hip_program_validate(buf, len(img), ctypes.byref(arena))
    # the schedule export decodes the same bytes: capacity probe, then a full plan
    n = ctypes.c_uint32()
    folded = (ctypes.c_int64 * 2)()
    lib.shk_hip_program_plan(buf, len(img), 0, None, None, folded, ctypes.byref(n))
    if n.value:
        streams = (ctypes.c_uint8 * n.value)()
        waits = (ctypes.c_int32 * n.value)()
        assert lib.shk_hip_program_plan(buf, len(img), n.value, streams, waits, folded,
                                        ctypes.byref(n)) == st
    return st


def main():
    rng = np.random.default_rng(1)
    good = images()
    for img in good:
        assert validate(img) == 0
    cases = 0
    hostile = [0, 1, 0x7FFFFFFF, 0xFFFFFFFF, 1 << 20, (1 << 20) + 1]
    for img in good:
        n = len(img)
        for cut in sorted(set([0, 1, 15, 16, 17, n // 2, n - 8, n - 1] +
                              list(rng.integers(0, n, 20)))):
            validate(img[:cut])
            cases += 1
        for _ in range(300):  # random bit flips
            b = bytearray(img)
            for _ in range(int(rng.integers(1, 4))):
                i = int(rng.integers(0, n))
                b[i] ^= 1 << int(rng.integers(0, 8))
            validate(bytes(b))
            cases += 1
        for _ in range(300):  # a hostile 32-bit or 64-bit value at a random aligned field
            b = bytearray(img)
            if rng.random() < 0.5:
                i = int(rng.integers(0, n // 4)) * 4
                b[i:i + 4] = struct.pack("<I", hostile[int(rng.integers(len(hostile)))])
            else:
                i = int(rng.integers(0, n // 8)) * 8
                v = [0, 1, -1, 1 << 40, -(1 << 62), (1 << 63) - 1][int(rng.integers(6))]
                b[i:i + 8] = struct.pack("<q", v)
            validate(bytes(b))
            cases += 1
    for _ in range(200):  # junk after a valid header
        hdr = struct.pack("<IIII", P.MAGIC, P.VERSION, int(rng.integers(0, 64)),
                          int(rng.integers(0, 64)))
        validate(hdr + rng.integers(0, 256, int(rng.integers(0, 4000)), dtype=np.uint8).tobytes())
        cases += 1
    # storage-transfer geometry
    for _ in range(3000):
        rank = int(rng.integers(0, 18))
        dims = [int(v) for v in rng.integers(-2, 6, rank)]
        strides = [int(v) for v in rng.integers(-3, 40, rank)] if rng.random() < 0.7 else None
        native.storage_transfer_bytes(int(rng.choice([1, 2, 3, 4, 8])), dims, strides,
                                      int(rng.integers(-2, 100)))
        cases += 1
    # LXM
    g = L64X128MixRandom(-7)
    g.next_longs(10_000)
    g.uniform_block(-1.0, 1.0, 10_000, np.float32)
    g.gaussian_block(100_000)  # fast path, overhangs, cap and tail
    from synaptik_amd.initializers import gaussian_tables
    gaussian_tables()
    # null and foreign handles
    vp = ctypes.c_void_p
    junk = vp(ctypes.addressof(ctypes.create_string_buffer(512)))
    assert lib.shk_hip_context_create(0, None) == 1
    for fn in ("shk_hip_context_release", "shk_hip_buffer_release", "shk_hip_program_release",
               "shk_hip_program_wait"):
        assert getattr(lib, fn)(None) == 1 and getattr(lib, fn)(junk) == 1
    out = vp()
    assert lib.shk_hip_buffer_create(junk, 64, ctypes.byref(out)) == 1 and not out.value
    assert lib.shk_hip_program_create(junk, b"x", 1, ctypes.byref(out)) == 1 and not out.value
    assert lib.shk_hip_program_run(junk, 0, None, 0, None) == 1
    assert lib.shk_hip_program_run_static(junk, 0, None, 0, None) == 1
    assert lib.shk_hip_program_validate(None, 0, None) == 1
    assert lib.shk_hip_program_plan(None, 0, 0, None, None, None, None) == 1
    for fn in ("shk_hip_program_set_graph_mode", "shk_hip_program_set_concurrent",
               "shk_hip_program_set_profiling"):
        assert getattr(lib, fn)(None, 1) == 1 and getattr(lib, fn)(junk, 0) == 1
    i32, u32, u64 = ctypes.c_int32(5), ctypes.c_uint32(5), ctypes.c_uint64(5)
    assert lib.shk_hip_program_graph_mode(junk, ctypes.byref(i32)) == 1 and i32.value == 0
    assert lib.shk_hip_program_graph_mode(junk, None) == 1
    for fn in ("shk_hip_program_side_steps", "shk_hip_program_step_count",
               "shk_hip_program_lease_count"):
        assert getattr(lib, fn)(junk, ctypes.byref(u32)) == 1
    assert lib.shk_hip_program_arena_bytes(junk, ctypes.byref(u64)) == 1
    msg = ctypes.create_string_buffer(64)
    assert lib.shk_hip_last_error(msg, 64) == 0
    assert lib.shk_hip_last_error(None, 0) == 1
    print(f"asan driver ok: {len(good)} images, {cases} malformed or random cases", flush=True)


if __name__ == "__main__":
    main()
