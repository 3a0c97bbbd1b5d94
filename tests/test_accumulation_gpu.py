"""Gradient accumulation modes on the device (GradientMode.java; TrainingParameter.stageAccumulation
:374-389; TrainingSessionTest.mapsMultipleParametersAndImplementsAccumulationAndZeroing)."""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.native import HipArithmeticError
from synaptik_amd.training import (Dense, GradientMode, HipTrainingSession, MlpSpec, Sgd,
                                   init_parameters)

pytestmark = pytest.mark.gpu


def _scalar(ctx, w0, lr):
    spec = MlpSpec([Dense(1, 1, None, bias=False)], "mse", "sum")
    return HipTrainingSession.open(ctx, spec, [np.array([[w0]], np.float32)], [None], Sgd(lr), 1)


def test_closed_form_accumulate_then_step(ctx):
    # (w*1 - 0)^2 from w = 2: gradient 4 per run; two accumulated runs, one step of lr 0.1
    s = _scalar(ctx, 2.0, 0.1)
    one, zero = np.array([[1.0]]), np.array([[0.0]])
    a = s.run(one, zero, GradientMode.ACCUMULATE)
    assert a.optimizer_step is None and a.accumulated_gradient_runs == 1
    assert s.state().weights[0][0, 0] == 2.0 and s.optimizer_steps == 0
    b = s.run(one, zero, GradientMode.ACCUMULATE_AND_STEP)
    assert b.optimizer_step == 1 and b.accumulated_gradient_runs == 0
    assert abs(s.state().weights[0][0, 0] - 1.2) <= 1e-6
    s.close()


def test_zero_grad_and_reset_ignore_pending(ctx):
    s = _scalar(ctx, 2.0, 0.1)
    one, zero = np.array([[1.0]]), np.array([[0.0]])
    s.run(one, zero, GradientMode.ACCUMULATE)
    s.zero_grad()
    assert s.accumulated_gradient_runs == 0
    s.run(one, zero, GradientMode.ACCUMULATE_AND_STEP)        # only this run's gradient 4
    assert abs(s.state().weights[0][0, 0] - 1.6) <= 1e-6
    s.run(one, zero, GradientMode.ACCUMULATE)                 # pending 2*1.6 = 3.2
    s.run(one, zero, GradientMode.RESET_AND_STEP)             # ignores and empties it
    assert abs(s.state().weights[0][0, 0] - (1.6 - 0.32)) <= 1e-6
    assert s.accumulated_gradient_runs == 0
    s.run(one, zero, GradientMode.ACCUMULATE_AND_STEP)        # accumulator was emptied
    w = 1.28
    assert abs(s.state().weights[0][0, 0] - (w - 0.2 * w)) <= 1e-6
    s.close()


def test_accumulated_step_matches_oracle(ctx):
    spec = MlpSpec.chain([16, 32, 4], hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 2, "he_normal")
    rng = np.random.default_rng(3)
    xa, xb = (rng.standard_normal((64, 16)).astype(np.float32) for _ in range(2))
    ya, yb = (rng.standard_normal((64, 4)).astype(np.float32) for _ in range(2))
    opt = Sgd(0.05, momentum=0.9)
    s = HipTrainingSession.open(ctx, spec, Ws, bs, opt, 64)
    s.run(xa, ya, GradientMode.ACCUMULATE)
    s.run(xb, yb, GradientMode.ACCUMULATE_AND_STEP)
    ref = oracle.OracleMLP(Ws, bs, ["relu", None], "mse", dict(kind="sgd", lr=0.05, momentum=0.9))
    _, gWa, gba, _ = ref.gradients(xa, ya)
    _, gWb, gbb, _ = ref.gradients(xb, yb)
    st = s.state()
    for got, p, ga, gb_ in zip(st.weights + st.biases, ref.W + ref.b, gWa + gba, gWb + gbb):
        summed = (ga + gb_).astype(np.float32)
        want, _ = oracle.sgd_stage(p, summed, np.zeros_like(p), lr=0.05, momentum=0.9)
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-5, atol=1e-7)
    s.close()


def test_non_finite_accumulation_commits_nothing(ctx):
    s = _scalar(ctx, 2.0, 0.1)
    one, zero = np.array([[1.0]]), np.array([[0.0]])
    s.run(one, zero, GradientMode.ACCUMULATE)
    acc_before = [a.download() for a in s.accum]
    with pytest.raises(HipArithmeticError):
        s.run(np.array([[1e30]]), zero, GradientMode.ACCUMULATE)   # gradient 2e60 -> inf
    assert s.accumulated_gradient_runs == 1
    assert all(np.array_equal(a.download(), b) for a, b in zip(s.accum, acc_before))
    s.run(one, zero, GradientMode.ACCUMULATE_AND_STEP)
    assert abs(s.state().weights[0][0, 0] - 1.2) <= 1e-6
    s.close()
