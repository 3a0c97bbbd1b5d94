"""Canonical host publication oracle (oracle.canonical_bytes, restating
MetalBackendRuntime.copyToCanonicalHostBytes, MetalBackendRuntime.java:360-398,489-499) pinned
against the reference's own known answers and against independent restatements: per-element
int.to_bytes(..., "big") over explicitly enumerated coordinates, and numpy's as_strided view
cast to a big-endian dtype."""
import itertools
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
UINT = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}


def raw_of(case):
    w = case["width"]
    return b"".join(int(h, 16).to_bytes(w, "little") for h in case["elements_hex"])


@pytest.mark.parametrize("case", GOLDEN["canonical_bytes"], ids=lambda c: c["source"][-12:] + c["dtype"])
def test_reference_known_answers(case):
    boolean = case["dtype"] == "BOOL"
    if "error" in case:
        with pytest.raises(ValueError):
            oracle.canonical_bytes(raw_of(case), case["width"], case["shape"], boolean=boolean)
    else:
        got = oracle.canonical_bytes(raw_of(case), case["width"], case["shape"], boolean=boolean)
        assert got.hex() == case["canonical_hex"]


def brute_force(raw, width, shape, strides, offset):
    """Independent restatement: enumerate coordinates with itertools.product (row-major order)."""
    out = bytearray()
    for coord in itertools.product(*[range(d) for d in shape]):
        e = offset + sum(c * s for c, s in zip(coord, strides))
        value = int.from_bytes(raw[e * width:(e + 1) * width], "little")
        out += value.to_bytes(width, "big")
    return bytes(out)


def dense_strides(shape):
    st, acc = [], 1
    for d in reversed(shape):
        st.append(acc)
        acc *= d
    return tuple(reversed(st))


VIEWS = [
    ((7,), None, 0),
    ((3, 5), None, 0),
    ((5, 3), (1, 5), 0),           # transpose of a [3,5] storage
    ((2, 3), (8, 2), 3),           # strided slice with an offset
    ((2, 3, 4), (0, 4, 1), 0),     # broadcast (stride 0) leading axis
    ((), None, 5),                 # rank-0 scalar at an offset
    ((1, 4, 1), (100, 3, 7), 2),
]


@pytest.mark.parametrize("width", [1, 2, 4, 8])
@pytest.mark.parametrize("view", VIEWS, ids=str)
def test_oracle_matches_brute_force(width, view):
    shape, strides, offset = view
    rng = np.random.default_rng(width * 31 + len(shape))
    raw = rng.integers(0, 256, 64 * 8, dtype=np.uint8).tobytes()
    st = strides if strides is not None else dense_strides(shape)
    want = brute_force(raw, width, shape, st, offset)
    assert oracle.canonical_bytes(raw, width, shape, strides, offset) == want


@pytest.mark.parametrize("width", [2, 4, 8])
def test_oracle_matches_numpy_big_endian_view(width):
    rng = np.random.default_rng(width)
    storage = rng.integers(0, 2 ** 63, 6 * 10, dtype=np.uint64).astype(UINT[width])
    view = np.lib.stride_tricks.as_strided(storage[2:], shape=(4, 6),
                                           strides=(10 * width, 1 * width))
    want = view.astype(np.dtype(UINT[width]).newbyteorder(">")).tobytes()
    got = oracle.canonical_bytes(storage.tobytes(), width, (4, 6), (10, 1), 2)
    assert got == want


def test_float_bits_kept():
    # NaN payloads, signed zero, subnormals and infinities keep their raw bits
    vals = np.array([0x7FC00123, 0x80000000, 0x00000001, 0x7F800000, 0xFF800000, 0x3F800000],
                    np.uint32)
    got = oracle.canonical_bytes(vals.tobytes(), 4, (6,))
    assert got == b"".join(int(v).to_bytes(4, "big") for v in vals)


def test_bool_validation_and_span():
    assert oracle.canonical_bytes(bytes([1, 0, 1]), 1, (3,), boolean=True) == bytes([1, 0, 1])
    with pytest.raises(ValueError):
        oracle.canonical_bytes(bytes([1, 255]), 1, (2,), boolean=True)
    # a non-canonical byte in a gap the view does not reference is not interpreted
    assert oracle.canonical_bytes(bytes([1, 7, 0]), 1, (2,), (2,), boolean=True) == bytes([1, 0])
    with pytest.raises(ValueError):
        oracle.canonical_bytes(bytes(8), 4, (3,))
