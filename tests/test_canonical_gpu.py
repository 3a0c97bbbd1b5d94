"""Canonical host publication on the device (shk_hip_buffer_download_canonical through the SPI
mirror HipBackendIntegration.copy_to_canonical_host_bytes) against the oracle restatement of
MetalBackendRuntime.copyToCanonicalHostBytes (MetalBackendRuntime.java:304-424): bit-exact."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.backend import HipBackendIntegration, TensorDescriptor

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
TYPE = {2: "FLOAT16", 4: "INT32", 8: "INT64"}


@pytest.fixture(scope="module")
def hip():
    integ = HipBackendIntegration.open(0)
    yield integ
    integ.close()


def upload_raw(hip, raw: bytes):
    return hip.borrow("BOOL", np.frombuffer(raw, np.uint8)) if raw else hip.borrow("BOOL", np.zeros(0, np.uint8))


@pytest.mark.parametrize("case", GOLDEN["canonical_bytes"], ids=lambda c: c["source"][-12:] + c["dtype"])
def test_reference_known_answers(hip, case):
    raw = b"".join(int(h, 16).to_bytes(case["width"], "little") for h in case["elements_hex"])
    buf = upload_raw(hip, raw)
    desc = TensorDescriptor(case["dtype"], tuple(case["shape"]))
    limit = case.get("maximum_bytes", len(raw))
    if "error" in case:
        with pytest.raises(ValueError):
            hip.copy_to_canonical_host_bytes(buf, desc, limit)
    else:
        assert hip.copy_to_canonical_host_bytes(buf, desc, limit).hex() == case["canonical_hex"]
    buf.close()


@pytest.mark.parametrize("width", [2, 4, 8])
@pytest.mark.parametrize("count", [1, 3, 4, 15, 17, 1000, 4097, 1 << 20])
def test_dense_matches_oracle(hip, width, count):
    rng = np.random.default_rng(count * 8 + width)
    raw = rng.integers(0, 256, count * width, dtype=np.uint8).tobytes()
    buf = upload_raw(hip, raw)
    got = hip.copy_to_canonical_host_bytes(buf, TensorDescriptor(TYPE[width], (count,)), count * width)
    assert got == oracle.canonical_bytes(raw, width, (count,))
    buf.close()


VIEWS = [
    ((5, 3), (1, 5), 0),
    ((2, 3), (8, 2), 3),
    ((2, 3, 4), (0, 4, 1), 0),
    ((), None, 5),
    ((1, 4, 1), (100, 3, 7), 2),
    ((33, 65), (1, 33), 0),
    ((7, 9), None, 11),
    ((1, 70, 1, 130), (5, 1, 9, 70), 3),   # transposed matrix with unit axes
    ((130, 64), (1, 200), 7),              # column slice of a wider storage
]


@pytest.mark.parametrize("width", [2, 4, 8])
@pytest.mark.parametrize("view", VIEWS, ids=str)
def test_strided_views_match_oracle(hip, width, view):
    shape, strides, offset = view
    rng = np.random.default_rng(width + len(shape))
    raw = rng.integers(0, 256, 16384 * width, dtype=np.uint8).tobytes()
    buf = upload_raw(hip, raw)
    count = int(np.prod(shape)) if shape else 1
    desc = TensorDescriptor(TYPE[width], shape, strides, offset)
    got = hip.copy_to_canonical_host_bytes(buf, desc, count * width)
    assert got == oracle.canonical_bytes(raw, width, shape, strides, offset)
    buf.close()


def test_bool_dense_strided_and_invalid(hip):
    rng = np.random.default_rng(5)
    vals = rng.integers(0, 2, 10007, dtype=np.uint8)
    buf = hip.borrow("BOOL", vals)
    assert hip.copy_to_canonical_host_bytes(buf, TensorDescriptor("BOOL", (10007,)), 10007) == vals.tobytes()
    bad = vals.copy()
    bad[9999] = 2  # in the tail after the last 16-byte chunk
    buf2 = hip.borrow("BOOL", bad)
    with pytest.raises(ValueError):
        hip.copy_to_canonical_host_bytes(buf2, TensorDescriptor("BOOL", (10007,)), 10007)
    bad2 = vals.copy()
    bad2[17] = 200  # inside a chunk
    buf3 = hip.borrow("BOOL", bad2)
    with pytest.raises(ValueError):
        hip.copy_to_canonical_host_bytes(buf3, TensorDescriptor("BOOL", (10007,)), 10007)
    # strided view that skips the bad byte is fine; one that reads it fails
    even = TensorDescriptor("BOOL", (5003,), (2,), 1)   # odd elements 1, 3, ..., 10005
    assert hip.copy_to_canonical_host_bytes(buf3, TensorDescriptor("BOOL", (5000,), (2,), 0), 5000) \
        == bad2[0:10000:2].tobytes()
    with pytest.raises(ValueError):
        hip.copy_to_canonical_host_bytes(buf3, even, 5003)
    for b in (buf, buf2, buf3):
        b.close()


def test_errors_follow_reference_order(hip):
    buf = hip.borrow("FLOAT32", np.arange(8, dtype=np.float32))
    with pytest.raises(ValueError, match="maximumBytes"):
        hip.copy_to_canonical_host_bytes(buf, TensorDescriptor("FLOAT32", (8,)), 31)
    with pytest.raises(ValueError, match="non-negative"):
        hip.copy_to_canonical_host_bytes(buf, TensorDescriptor("FLOAT32", (8,)), -1)
    with pytest.raises(ValueError):  # span beyond the buffer
        hip.copy_to_canonical_host_bytes(buf, TensorDescriptor("FLOAT32", (9,)), 1 << 20)
    with pytest.raises(ValueError):
        hip.copy_to_canonical_host_bytes(buf, TensorDescriptor("FLOAT32", (4,), (2,), 2), 1 << 20)
    for fp8 in ("FLOAT8_E4M3", "FLOAT8_E5M2"):
        with pytest.raises(ValueError):
            hip.copy_to_canonical_host_bytes(buf, TensorDescriptor(fp8, (8,)), 8)
        with pytest.raises(ValueError):
            hip.borrow(fp8, np.zeros(2, np.uint8))
    assert hip.copy_to_canonical_host_bytes(buf, TensorDescriptor("FLOAT32", (0, 3)), 0) == b""
    buf.close()


def test_full_size_c4_output_round_trip(hip):
    """[4096, 4096] FLOAT32 (the MLP-4096 output): big-endian decode recovers every raw bit, and
    the transposed view equals numpy's transpose."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4096, 4096)).astype(np.float32)
    x[0, :4] = [np.nan, -0.0, np.inf, 1e-45]
    buf = hip.borrow("FLOAT32", x)
    got = hip.copy_to_canonical_host_bytes(buf, TensorDescriptor("FLOAT32", x.shape), x.nbytes)
    assert np.array_equal(np.frombuffer(got, ">u4").reshape(x.shape), x.view(np.uint32))
    t = hip.copy_to_canonical_host_bytes(buf, TensorDescriptor("FLOAT32", (4096, 4096), (1, 4096)),
                                         x.nbytes)
    assert np.array_equal(np.frombuffer(t, ">u4").reshape(x.shape), x.view(np.uint32).T)
    buf.close()
