"""The optimizer update fused into the weight-gradient GEMM epilogue against the streaming pass.

The fused path runs the same per-element SGD / Adam / AdamW arithmetic (TrainingParameter.java:
433-525, 622-672) on the same binary32 gradient, so parameters and slots must agree bit for bit
with the unfused program (gradient stored, then the staged optimizer pass) over several steps,
for every epilogue that can carry it: the MFMA tile epilogue, the split-K reduction and the
K == 1 outer product. The unfused program is itself checked against the oracle elsewhere.
"""
import numpy as np
import pytest

from synaptik_amd import training
from synaptik_amd.native import HipArithmeticError
from synaptik_amd.training import Adam, AdamW, Dense, HipTrainingSession, MlpSpec, Sgd, init_parameters

pytestmark = pytest.mark.gpu

OPTIMIZERS = [
    Sgd(0.05),
    Sgd(0.05, momentum=0.9, nesterov=True, weight_decay=0.01),
    Sgd(0.05, momentum=0.5, dampening=0.3, weight_decay=0.001),
    Adam(1e-2, 0.9, 0.999, 1e-8, weight_decay=0.01),
    AdamW(1e-2, 0.9, 0.999, 1e-8, 0.01),
]

# (widths, batch): MFMA epilogue (odd extents, partial tiles); split-K reduction (few output
# tiles, long batch); K == 1 (one row); the large-problem kernel (first layer's 2048x2048
# weight gradient, and a 2100x2000 one with ragged 128-wide tiles, whose update loads go a
# chunk of row steps ahead with the rows past the edge masked)
SHAPES = [([37, 130, 67, 3], 96), ([64, 96, 32, 1], 4096), ([16, 24, 8, 1], 1),
          ([2048, 2048, 8], 64), ([784, 1024, 8], 1024), ([784, 1024, 10], 1024),
          ([2000, 2100, 8], 64)]


def _run(ctx, monkeypatch, fuse, spec, Ws, bs, opt, x, y, steps):
    monkeypatch.setattr(training, "FUSE_OPTIMIZER", fuse)
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, opt, x.shape[0])
    losses = [sess.run(x, y).objective for _ in range(steps)]
    st = sess.state()
    sess.close()
    return losses, st


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("shape", SHAPES, ids=["tile", "splitk", "k1", "large", "edge64", "classifier",
                                                 "large_ragged"])
@pytest.mark.parametrize("opt", OPTIMIZERS, ids=["sgd", "nesterov", "dampening", "adam", "adamw"])
def test_fused_update_matches_streaming_pass(ctx, monkeypatch, shape, opt):
    widths, batch = shape
    spec = MlpSpec.chain(widths, hidden="tanh", loss="mse")
    Ws, bs = init_parameters(spec, 11, "xavier_uniform")
    rng = np.random.default_rng(4)
    x = rng.standard_normal((batch, widths[0])).astype(np.float32)
    y = rng.standard_normal((batch, widths[-1])).astype(np.float32)
    la, a = _run(ctx, monkeypatch, True, spec, Ws, bs, opt, x, y, 4)
    lb, b = _run(ctx, monkeypatch, False, spec, Ws, bs, opt, x, y, 4)
    assert la == lb
    assert a.optimizer_steps == b.optimizer_steps == 4
    for t in ("weights", "biases", "first", "second"):
        for u, v in zip(getattr(a, t), getattr(b, t)):
            assert np.array_equal(_bits(u), _bits(v)), t


def test_fused_update_without_biases_flags_failures(ctx, monkeypatch):
    """With no bias tensors every update runs in a GEMM epilogue: a non-finite candidate must
    still fail the run and commit nothing."""
    monkeypatch.setattr(training, "FUSE_OPTIMIZER", True)
    spec = MlpSpec([Dense(4, 8, "relu", bias=False), Dense(8, 1, None, bias=False)], "mse")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), 8)
    x = np.ones((8, 4), np.float32)
    sess.run(x, np.zeros((8, 1), np.float32))
    before = sess.state()
    with pytest.raises(HipArithmeticError):
        sess.run(x, np.full((8, 1), 3e38, np.float32))
    after = sess.state()
    assert after.optimizer_steps == before.optimizer_steps == 1
    for u, v in zip(before.weights + before.first + before.second,
                    after.weights + after.first + after.second):
        assert np.array_equal(_bits(u), _bits(v))
    sess.run(x, np.zeros((8, 1), np.float32))
    assert sess.optimizer_steps == 2
    sess.close()
