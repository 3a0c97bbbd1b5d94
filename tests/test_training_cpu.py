"""Host-side checks of the training session that need no device: batch validation
(check_batch) rejects what the reference rejects before any work is done."""
import numpy as np
import pytest

from synaptik_amd.training import MlpSpec, check_batch


def _mse():
    return MlpSpec.chain([4, 8, 3], hidden="relu", loss="mse")


def _ce():
    return MlpSpec.chain([4, 8, 10], hidden="relu", loss="ce")


def test_accepts_matching_batches_and_converts():
    x, y = check_batch(_mse(), 6, "i64", np.ones((6, 4)), np.zeros((6, 3), np.int32))
    assert x.dtype == np.float32 and x.flags.c_contiguous and x.shape == (6, 4)
    assert y.dtype == np.float32 and y.shape == (6, 3)
    x, y = check_batch(_ce(), 6, "i64", np.ones((6, 4), np.float32), np.arange(6, dtype=np.int32))
    assert y.dtype == np.int64 and np.array_equal(y, np.arange(6))
    _, y = check_batch(_ce(), 6, "i32", np.ones((6, 4), np.float32), np.arange(6))
    assert y.dtype == np.int32
    # a transposed (non-contiguous) view is accepted and packed
    x, _ = check_batch(_mse(), 4, "i64", np.ones((4, 4)).T, np.zeros((4, 3)))
    assert x.flags.c_contiguous


@pytest.mark.parametrize("x,y", [
    (np.ones((5, 4)), np.zeros((5, 3))),            # short batch
    (np.ones((6, 5)), np.zeros((6, 3))),            # wrong fan_in
    (np.ones((6, 4)), np.zeros((6, 2))),            # wrong fan_out
    (np.ones((6, 4)), np.zeros(18)),                # flat target
    (np.ones(24), np.zeros((6, 3))),                # flat input
    (np.ones((6, 4)).astype(object), np.zeros((6, 3))),
], ids=["short", "fan-in", "fan-out", "flat-y", "flat-x", "object"])
def test_mse_mismatches_raise(x, y):
    with pytest.raises(ValueError):
        check_batch(_mse(), 6, "i64", x, y)


@pytest.mark.parametrize("y,dt", [
    (np.zeros(5, np.int64), "i64"),                  # short
    (np.zeros((6, 1), np.int64), "i64"),             # not rank 1
    (np.zeros(6, np.float32), "i64"),                # float labels
    (np.array([0, 1, 2, 3, 4, 2**31], np.int64), "i32"),   # does not fit INT32
    (np.array([0, 1, 2, 3, 4, 2**63], np.uint64), "i64"),  # does not fit INT64
], ids=["short", "rank", "float", "i32-range", "i64-range"])
def test_ce_label_mismatches_raise(y, dt):
    with pytest.raises(ValueError):
        check_batch(_ce(), 6, dt, np.ones((6, 4)), y)
