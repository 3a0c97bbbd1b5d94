"""CPU<->HIP prepared storage-layout transfers on the device (shk_hip_buffer_upload_storage /
shk_hip_buffer_download_storage through HipBackendIntegration.bind_storage_layout_* and
CpuHipPreparedBufferTransfer), modelled on the reference's MetalMpsGraphAffineNativeTest.java:
290-410 and MetalBackendRuntime.java:211-281: the physical span moves byte for byte (prefix and
gap bytes included), BOOL logical elements are validated before anything is written, and
mismatched sizes or geometries are refused."""
import json
from pathlib import Path

import numpy as np
import pytest

from synaptik_amd.backend import (CpuHipPreparedBufferTransfer, HipBackendIntegration,
                                  TensorDescriptor)

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
# bit patterns that a float round trip would disturb: NaN payloads, signed zero, subnormal, inf
ADVERSARIAL = np.array([0x7FC00123, 0x80000000, 0x00000001, 0x7F800000, 0xFF800001, 0x3F800000,
                        0x7FBFFFFF, 0x80800000], np.uint32)


@pytest.fixture(scope="module")
def hip():
    integ = HipBackendIntegration.open(0)
    yield integ
    integ.close()


def test_select_download_covers_prefix_bytes(hip):
    # MetalMpsGraphAffineNativeTest.java:293-313: [4] at offset 4 over 8 storage elements
    storage = np.where(np.arange(8) < 4, np.uint32(0x5A5A5A5A), ADVERSARIAL).astype(np.uint32)
    buf = hip.borrow("FLOAT32", storage)
    d = TensorDescriptor("FLOAT32", (4,), (1,), 4)
    assert hip.accepts_storage_layout_transfer(buf, d)
    out = np.zeros(8, np.uint32)
    hip.bind_storage_layout_download(buf, d)(out)
    assert np.array_equal(out, storage)
    buf.close()


def test_slice_upload_replaces_the_whole_span(hip):
    # MetalMpsGraphAffineNativeTest.java:315-344: [2,2] strides [8,2] offset 5, 16 elements
    storage = np.full(16, 0x6B6B6B6B, np.uint32)
    storage[[5, 7, 13, 15]] = ADVERSARIAL[:4]
    replacement = (0x7C7C7C7C + np.arange(16)).astype(np.uint32)
    buf = hip.borrow("FLOAT32", storage)
    d = TensorDescriptor("FLOAT32", (2, 2), (8, 2), 5)
    assert hip.accepts_storage_layout_transfer(buf, d)
    hip.bind_storage_layout_upload(buf, d)(replacement)
    out = np.zeros(16, np.uint32)
    hip.bind_storage_layout_download(buf, d)(out)
    assert np.array_equal(out, replacement)
    buf.close()


@pytest.mark.parametrize("case", GOLDEN["storage_transfer"], ids=lambda c: c["source"][-9:])
def test_reference_cases_on_a_live_buffer(hip, case):
    d = TensorDescriptor(case["dtype"], tuple(case["shape"]),
                         None if case["strides"] is None else tuple(case["strides"]),
                         case["offset"], case.get("resolved", True))
    width = {"FLOAT32": 4, "FLOAT64": 8}[case["dtype"]]
    span = case.get("span", 1)
    buf = hip.borrow(case["dtype"], np.zeros(span * width, np.uint8))
    assert hip.accepts_storage_layout_transfer(buf, d) == case["supports"]
    if not case["supports"]:
        with pytest.raises(ValueError):
            hip.bind_storage_layout_download(buf, d)
        with pytest.raises(ValueError):
            hip.bind_storage_layout_upload(buf, d)
    buf.close()


def test_size_mismatches_are_refused(hip):
    d = TensorDescriptor("FLOAT32", (3, 5))
    big = hip.borrow("FLOAT32", np.zeros(16, np.float32))      # 64 bytes, extent is 60
    assert not hip.accepts_storage_layout_transfer(big, d)
    with pytest.raises(ValueError):
        hip.bind_storage_layout_upload(big, d)
    big.close()
    buf = hip.borrow("FLOAT32", np.zeros(15, np.float32))
    up = hip.bind_storage_layout_upload(buf, d)
    with pytest.raises(ValueError):
        up(np.zeros(14, np.float32))                             # host source too small
    down = hip.bind_storage_layout_download(buf, d)
    with pytest.raises(ValueError):
        down(np.zeros(14, np.float32))
    buf.close()


def test_bool_upload_validates_logical_elements_only(hip):
    d = TensorDescriptor("BOOL", (2, 3), (8, 2), 1)               # logical bytes 1,3,5,9,11,13
    span = 14
    buf = hip.borrow("BOOL", np.zeros(span, np.uint8))
    up = hip.bind_storage_layout_upload(buf, d)
    src = np.zeros(span, np.uint8)
    src[[1, 5, 11]] = 1
    src[[0, 2, 4, 12]] = 0xEE                                     # gaps: not interpreted
    up(src)
    out = np.zeros(span, np.uint8)
    hip.bind_storage_layout_download(buf, d)(out)
    assert np.array_equal(out, src)
    bad = src.copy()
    bad[9] = 2                                                    # a logical element
    with pytest.raises(ValueError, match="non-canonical"):
        up(bad)
    hip.bind_storage_layout_download(buf, d)(out)
    assert np.array_equal(out, src)                               # device untouched
    buf.close()


def test_bool_download_fails_before_writing(hip):
    d = TensorDescriptor("BOOL", (4, 3), (1, 4), 0)                # transposed, 12 elements
    raw = np.tile(np.array([0, 1], np.uint8), 6)
    raw[7] = 3
    buf = hip.borrow("BOOL", raw)
    out = np.full(12, 0xAB, np.uint8)
    with pytest.raises(ValueError, match="non-canonical"):
        hip.bind_storage_layout_download(buf, d)(out)
    assert np.all(out == 0xAB)
    buf.close()


@pytest.mark.parametrize("dtype,np_t", [("FLOAT64", np.uint64), ("FLOAT16", np.uint16),
                                        ("INT32", np.uint32), ("BOOL", np.uint8)])
def test_prepared_transfer_round_trip(hip, dtype, np_t):
    rng = np.random.default_rng(3)
    shape, strides, offset = (37, 19), (1, 41), 6                # column-major with gaps
    d = TensorDescriptor(dtype, shape, strides, offset)
    extent = CpuHipPreparedBufferTransfer.supports(d) and hip.storage_transfer_extent(d)
    assert extent
    n = extent // np.dtype(np_t).itemsize
    host = (rng.integers(0, 2, n) if dtype == "BOOL" else
            rng.integers(0, np.iinfo(np_t).max, n, dtype=np_t, endpoint=True)).astype(np_t)
    dev = hip.borrow(dtype, np.zeros(n, np_t))
    up = CpuHipPreparedBufferTransfer.cpu_to_hip(hip, extent, d)
    down = CpuHipPreparedBufferTransfer.hip_to_cpu(hip, extent, d)
    back = np.zeros(n, np_t)
    up.bind(host, dev).execute()
    down.bind(dev, back).execute()
    assert np.array_equal(back, host)
    with pytest.raises(ValueError):
        CpuHipPreparedBufferTransfer.cpu_to_hip(hip, extent + 1, d)
    with pytest.raises(ValueError):
        down.bind(dev, np.zeros(n, np_t)[::-1])                  # not C-contiguous
    with pytest.raises(ValueError):
        down.bind(dev, np.zeros(n, np_t).view()[:-1])
    ro = np.zeros(n, np_t)
    ro.flags.writeable = False
    with pytest.raises(ValueError):
        down.bind(dev, ro)
    dev.close()


def test_large_transfer_round_trip(hip):
    # 256 MiB of FLOAT32 storage, a [8192, 8192] row slice of a wider matrix
    d = TensorDescriptor("FLOAT32", (8192, 8000), (8192, 1), 0)
    extent = hip.storage_transfer_extent(d)
    n = extent // 4
    host = np.random.default_rng(5).integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    dev = hip.borrow("FLOAT32", np.zeros(n, np.uint32))
    CpuHipPreparedBufferTransfer.cpu_to_hip(hip, extent, d).bind(host, dev).execute()
    back = np.empty(n, np.uint32)
    CpuHipPreparedBufferTransfer.hip_to_cpu(hip, extent, d).bind(dev, back).execute()
    assert np.array_equal(back, host)
    dev.close()
