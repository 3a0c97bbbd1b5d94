"""Storage-layout transfer geometry (CPU/HIP prepared buffer transfers).

The oracle's storage_transfer_bytes restates MetalBackendRuntime.isStorageTransfer /
CpuMetalPreparedBufferTransfer.transferByteCount; it is pinned here against the reference's own
cases (tests/golden/reference_known_answers.json, "storage_transfer") and against what the
rule has to guarantee, checked by enumeration on small views: an accepted view maps distinct
coordinates to distinct storage elements, its highest element is span - 1, and every axis
permutation of a dense layout (with or without gaps between axes) is accepted. The native host
function behind the product (shk_hip_storage_transfer_bytes) must then agree with the oracle on
every case, including the overflow edges."""
import itertools
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.backend import (CpuHipPreparedBufferTransfer, STORAGE_WIDTH, TensorDescriptor,
                                  storage_transfer_extent)
from synaptik_amd.native import storage_transfer_bytes

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
LONG_MAX = (1 << 63) - 1


def descriptor(case):
    return TensorDescriptor(case["dtype"], tuple(case["shape"]),
                            None if case["strides"] is None else tuple(case["strides"]),
                            case["offset"], case.get("resolved", True))


@pytest.mark.parametrize("case", GOLDEN["storage_transfer"], ids=lambda c: c["source"][-9:])
def test_reference_cases(case):
    d = descriptor(case)
    w = STORAGE_WIDTH[case["dtype"]]
    want = case["span"] * w if case["supports"] else 0
    if case.get("resolved", True):
        assert oracle.storage_transfer_bytes(w, d.shape, d.strides, d.storage_offset) == want
    assert storage_transfer_extent(d) == want
    assert CpuHipPreparedBufferTransfer.supports(d) == case["supports"]


def addresses(shape, strides, offset):
    return [offset + sum(c * s for c, s in zip(coord, strides))
            for coord in itertools.product(*[range(d) for d in shape])]


def test_accepted_views_are_injective_with_the_stated_span():
    rng = np.random.default_rng(7)
    accepted = rejected_overlapping = 0
    for _ in range(6000):
        rank = int(rng.integers(0, 5))
        shape = [int(x) for x in rng.integers(1, 5, rank)]
        strides = [int(x) for x in rng.integers(1, 13, rank)]
        offset = int(rng.integers(0, 6))
        got = oracle.storage_transfer_bytes(4, shape, strides, offset)
        a = addresses(shape, strides, offset)
        if got:
            accepted += 1
            assert len(set(a)) == len(a), (shape, strides)
            assert got == (max(a) + 1) * 4, (shape, strides, offset)
        else:
            rejected_overlapping += len(set(a)) < len(a)
    assert accepted > 300 and rejected_overlapping > 300


@pytest.mark.parametrize("shape", [(3, 4), (2, 3, 5), (1, 4, 1, 2), (5,)])
def test_every_permutation_of_a_dense_layout_with_gaps_is_accepted(shape):
    for perm in itertools.permutations(range(len(shape))):
        for gap in (0, 1, 3):
            # lay the axes out in the order `perm` (last fastest) with `gap` spare elements
            strides = [0] * len(shape)
            e = 1
            for a in reversed(perm):
                strides[a] = e
                e = e * shape[a] + gap
            got = oracle.storage_transfer_bytes(2, shape, strides, 3)
            a = addresses(shape, strides, 3)
            assert got == (max(a) + 1) * 2, (shape, perm, gap)


def test_overlap_and_degenerate_views_are_rejected():
    assert oracle.storage_transfer_bytes(4, (2, 3), (2, 1), 0) == 0          # rows overlap
    assert oracle.storage_transfer_bytes(4, (3, 3), (1, 1), 0) == 0
    assert oracle.storage_transfer_bytes(4, (2, 2), (3, 2), 0) != 0          # interleaved, no overlap
    assert oracle.storage_transfer_bytes(4, (2,), (-1,), 1) == 0
    assert oracle.storage_transfer_bytes(4, (), None, 0) == 4                 # scalar: one element
    assert oracle.storage_transfer_bytes(4, (), None, 9) == 40
    assert oracle.storage_transfer_bytes(8, (1,), (1,), LONG_MAX // 8 - 1) == (LONG_MAX // 8) * 8
    assert oracle.storage_transfer_bytes(8, (1,), (1,), LONG_MAX // 8) == 0
    assert oracle.storage_transfer_bytes(4, [1] * 17, None, 0) == 0           # rank > 16


def test_native_matches_the_oracle():
    rng = np.random.default_rng(11)
    cases = []
    for _ in range(4000):
        rank = int(rng.integers(0, 6))
        shape = [int(x) for x in rng.integers(0, 6, rank)]
        strides = [int(x) for x in rng.integers(-1, 40, rank)]
        cases.append((int(rng.choice([1, 2, 4, 8])), shape,
                      None if rng.random() < 0.2 else strides, int(rng.integers(-1, 50))))
    big = [1 << 30, 1 << 31, 1 << 40, (1 << 62) // 3, 1 << 62, LONG_MAX // 2, LONG_MAX]
    for _ in range(3000):
        rank = int(rng.integers(1, 4))
        shape = [int(rng.choice(big + [1, 2, 3])) for _ in range(rank)]
        strides = [int(rng.choice(big + [1, 2, 7])) for _ in range(rank)]
        cases.append((int(rng.choice([1, 2, 4, 8])), shape, strides,
                      int(rng.choice([0, 5, LONG_MAX - 1, LONG_MAX // 8]))))
    for w, shape, strides, off in cases:
        want = oracle.storage_transfer_bytes(w, shape, strides, off)
        assert storage_transfer_bytes(w, shape, strides, off) == want, (w, shape, strides, off)


def test_fp8_and_unresolved_layouts_are_not_transfers():
    assert storage_transfer_extent(TensorDescriptor("FLOAT8_E4M3", (4,))) == 0
    assert storage_transfer_extent(TensorDescriptor("FLOAT32", (4,), layout_resolved=False)) == 0
    assert storage_transfer_extent(TensorDescriptor("BOOL", (4,))) == 4
