"""The fused classifier head (one step: logits, index cross-entropy, logit and input cotangents)
against the unfused lowering (row-dot GEMM, CE pass 1 and gradient, small-K GEMM): every
objective, parameter and optimizer slot bit-identical after each step, over class counts in every
compiled bucket, ragged batches, widths that take the scalar path, both label widths, each
hidden activation and a head with no hidden layer. The unfused lowering is itself pinned against
the oracle (test_training_gpu.py, test_configs_full_gpu.py)."""
import numpy as np
import pytest

import synaptik_amd.training as training
from synaptik_amd.native import HipIndexError
from synaptik_amd.program import OP_CE_HEAD, OP_CE_INDEX
from synaptik_amd.training import (Adam, HipTrainingSession, MlpSpec, Sgd, init_parameters,
                                   lower_training_step)

pytestmark = pytest.mark.gpu


def _session(ctx, spec, opt, batch, fused, label_dtype="i64", seed=0):
    Ws, bs = init_parameters(spec, seed, "he_normal")
    old = training.FUSE_CE_HEAD
    training.FUSE_CE_HEAD = fused
    try:
        sess = HipTrainingSession.open(ctx, spec, Ws, bs, opt, batch, label_dtype=label_dtype)
    finally:
        training.FUSE_CE_HEAD = old
    return sess


def _assert_state_identical(a, b):
    sa, sb = a.state(), b.state()
    for name in ("weights", "biases", "first", "second"):
        for u, v in zip(getattr(sa, name), getattr(sb, name)):
            assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), name
    assert sa.optimizer_steps == sb.optimizer_steps


CASES = [
    # widths, hidden activation, batch, optimizer
    ([784, 1024, 1024, 10], "relu", 1024, "adam"),   # the C3 classifier
    ([64, 48, 3], "tanh", 37, "sgd"),                 # ragged batch (not a multiple of 4 rows)
    ([32, 40, 16], "sigmoid", 64, "adam"),            # 16 classes: the largest bucket
    ([30, 21, 2], "relu", 9, "sgd"),                  # head width off 4: the scalar path
    ([64, 2048, 10], "relu", 12, "adam"),             # W over 64 KB: read from L2, not LDS
    ([20, 1], None, 16, "sgd"),                       # no hidden layer: no input cotangent
    ([24, 32, 32, 5], "relu", 128, "adam"),
]


@pytest.mark.parametrize("widths,act,batch,opt", CASES)
@pytest.mark.parametrize("label_dtype", ["i64", "i32"])
def test_fused_head_matches_unfused_lowering_bit_for_bit(ctx, widths, act, batch, opt, label_dtype):
    print(f"[ce_head] widths={widths} act={act} batch={batch} opt={opt} labels={label_dtype}",
          flush=True)
    spec = MlpSpec.chain(widths, hidden=act or "relu", loss="ce")
    make_opt = (lambda: Adam(1e-3, 0.9, 0.999, 1e-8)) if opt == "adam" else (
        lambda: Sgd(0.05, momentum=0.9))
    # the program really is fused / unfused
    pb, _ = lower_training_step(spec, batch, make_opt(), label_dtype=label_dtype)
    ops = [s.opcode for s in pb.steps]
    assert ops.count(OP_CE_HEAD) == 2 and OP_CE_INDEX not in ops
    fused = _session(ctx, spec, make_opt(), batch, True, label_dtype)
    plain = _session(ctx, spec, make_opt(), batch, False, label_dtype)
    rng = np.random.default_rng(batch)
    for step in range(3):
        x = rng.standard_normal((batch, widths[0])).astype(np.float32)
        y = rng.integers(0, widths[-1], batch).astype(np.int64 if label_dtype == "i64" else np.int32)
        a = fused.run(x, y).objective
        b = plain.run(x, y).objective
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), step
        _assert_state_identical(fused, plain)
    fused.close()
    plain.close()


def test_fused_head_rejects_out_of_range_targets_and_keeps_state(ctx):
    spec = MlpSpec.chain([16, 24, 4], hidden="relu", loss="ce")
    sess = _session(ctx, spec, Sgd(0.1), 8, True)
    before = sess.state()
    x = np.ones((8, 16), np.float32)
    for bad in (4, -1):
        y = np.zeros(8, np.int64)
        y[5] = bad
        with pytest.raises(HipIndexError):
            sess.run(x, y)
        after = sess.state()
        for u, v in zip(before.weights + before.biases, after.weights + after.biases):
            assert np.array_equal(u, v)
    sess.run(x, np.zeros(8, np.int64))  # a valid batch still runs
    sess.close()


@pytest.mark.parametrize("concurrent", [True, False])
def test_loss_mean_folded_into_publication_matches_its_own_launch(ctx, concurrent):
    """Unprofiled runs perform the fused head's loss MEAN inside the run's publication kernel;
    profiled runs launch it as a step of its own. Both give the same objective after every step
    and the same parameters and slots, on the two-stream schedule and on one stream."""
    spec = MlpSpec.chain([784, 1024, 1024, 10], hidden="relu", loss="ce")
    rng = np.random.default_rng(61)
    x = rng.uniform(0, 1, (1024, 784)).astype(np.float32)
    y = rng.integers(0, 10, 1024).astype(np.int64)
    a = _session(ctx, spec, Adam(1e-3, 0.9, 0.999, 1e-8), 1024, True)
    b = _session(ctx, spec, Adam(1e-3, 0.9, 0.999, 1e-8), 1024, True)
    for sess in (a, b):
        for prog, _ in sess._programs.values():
            prog.set_concurrent(concurrent)
    for prog, _ in b._programs.values():
        prog.set_profiling(True)
    for step in range(4):
        la = a.run(x, y).objective
        lb = b.run(x, y).objective
        print(f"fold step={step} concurrent={concurrent} {la} {lb}", flush=True)
        assert np.float32(la).view(np.uint32) == np.float32(lb).view(np.uint32)
    _assert_state_identical(a, b)
    a.close()
    b.close()
