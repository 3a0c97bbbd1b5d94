"""Training-step parity on the GPU against the oracle's composition of the reference algorithms.

Configurations follow the benchmark set: C1 (16->64->1 tanh, MSE, SGD 0.01, batch 256, 20 steps; loss
trajectory within 1e-4 relative) and the C3 classifier architecture (784->1024->1024->10 ReLU,
index softmax-CE, Adam) at a reduced batch so the oracle finishes in seconds. Closed-form known
answers come from the reference's own tests.
"""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.native import HipArithmeticError, HipIndexError
from synaptik_amd.training import (Adam, AdamW, Dense, HipTrainingSession, MlpSpec, Sgd,
                                   init_parameters, lower_training_step)
from tests.conftest import needs_fold, needs_two_streams

pytestmark = pytest.mark.gpu


def _c1_data():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((256, 16)).astype(np.float32)
    y = (np.sin(x.astype(np.float64)).sum(1, keepdims=True)
         + 0.01 * rng.standard_normal((256, 1))).astype(np.float32)
    return x, y


def test_c1_twenty_step_loss_trajectory(ctx):
    spec = MlpSpec.chain([16, 64, 1], hidden="tanh", loss="mse")
    Ws, bs = init_parameters(spec, 0, "builder")  # Model.builder().seed(0)
    x, y = _c1_data()
    ref = oracle.OracleMLP(Ws, bs, ["tanh", None], "mse", dict(kind="sgd", lr=0.01))
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.01), 256)
    got, want = [], []
    for _ in range(20):
        got.append(sess.run(x, y).objective)
        want.append(float(ref.step(x, y)))
    np.testing.assert_allclose(got, want, rtol=1e-4)
    assert got[-1] < got[0]
    st = sess.state()
    assert st.optimizer_steps == 20
    for a, b in zip(st.weights + st.biases, ref.W + ref.b):
        np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-6)
    sess.close()


@pytest.mark.parametrize("opt", [
    Sgd(0.05, momentum=0.9),
    Sgd(0.05, momentum=0.9, nesterov=True, weight_decay=0.01),
    Sgd(0.05, momentum=0.5, dampening=0.3, weight_decay=0.001),
])
def test_sgd_variants_against_oracle(ctx, opt):
    spec = MlpSpec.chain([16, 64, 32, 1], hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 3, "he_normal")
    x, y = _c1_data()
    ref = oracle.OracleMLP(Ws, bs, ["relu", "relu", None], "mse",
                           dict(kind="sgd", lr=opt.learning_rate, momentum=opt.momentum,
                                dampening=opt.dampening, weight_decay=opt.weight_decay,
                                nesterov=opt.nesterov))
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, opt, 256)
    for _ in range(5):
        np.testing.assert_allclose(sess.run(x, y).objective, float(ref.step(x, y)), rtol=1e-4)
    st = sess.state()
    for a, b in zip(st.first, ref.m):
        np.testing.assert_allclose(a.ravel(), b.ravel(), rtol=1e-3, atol=1e-6)
    sess.close()


@pytest.mark.parametrize("opt", [Adam(1e-3, 0.9, 0.999, 1e-8), AdamW(1e-3, 0.9, 0.999, 1e-8, 0.01)])
def test_c3_classifier_architecture_adam(ctx, opt):
    batch = 64
    spec = MlpSpec.chain([784, 1024, 1024, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 1, "he_normal")
    rng = np.random.default_rng(2)
    x = rng.uniform(0, 1, size=(batch, 784)).astype(np.float32)
    labels = rng.integers(0, 10, size=batch).astype(np.int64)
    ref = oracle.OracleMLP(Ws, bs, ["relu", "relu", None], "ce",
                           dict(kind="adamw" if opt.decoupled else "adam", lr=opt.learning_rate,
                                beta1=opt.beta1, beta2=opt.beta2, eps=opt.epsilon,
                                weight_decay=opt.weight_decay))
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, opt, batch)
    got, want = [], []
    for _ in range(4):
        got.append(sess.run(x, labels).objective)
        want.append(float(ref.step(x, labels)))
    np.testing.assert_allclose(got, want, rtol=1e-4)
    st = sess.state()
    for a, b in zip(st.weights, ref.W):
        rel = np.linalg.norm(a - b) / np.linalg.norm(b)
        assert rel < 1e-5
    sess.close()


def _scalar_session(ctx, w0, opt, reduction="mean"):
    spec = MlpSpec([Dense(1, 1, None, bias=False)], "mse", reduction)
    return HipTrainingSession.open(ctx, spec, [np.array([[w0]], np.float32)], [None], opt, 1)


def test_known_answer_scalar_sgd(ctx):
    """TrainingSessionCpuIntegrationTest.freshValuesTrainOnCpu (:48-92): objective 25 then 1,
    weight 2 -> -1 -> -1.4 with Sgd(0.1)."""
    sess = _scalar_session(ctx, 2.0, Sgd(0.1))
    s1 = sess.run(np.array([[3.0]]), np.array([[1.0]]))
    assert s1.objective == 25.0
    assert abs(sess.state().weights[0][0, 0] - (-1.0)) <= 1e-6
    s2 = sess.run(np.array([[2.0]]), np.array([[-3.0]]))
    assert abs(s2.objective - 1.0) <= 1e-6
    assert abs(sess.state().weights[0][0, 0] - (-1.4)) <= 1e-6
    assert sess.optimizer_steps == 2


def test_known_answer_sgd_momentum(ctx):
    """TrainingSessionTest (:215-240): (w - 0)^2 from w = 2 with Sgd(0.1, momentum 0.5):
    objective 4, w = 1.6, then w = 1.08 with momentum slot 5.2."""
    sess = _scalar_session(ctx, 2.0, Sgd(0.1, momentum=0.5))
    one, zero = np.array([[1.0]]), np.array([[0.0]])
    assert sess.run(one, zero).objective == 4.0
    assert abs(sess.state().weights[0][0, 0] - 1.6) <= 1e-6
    sess.run(one, zero)
    st = sess.state()
    assert abs(st.weights[0][0, 0] - 1.08) <= 1e-6
    assert abs(st.first[0][0] - 5.2) <= 1e-6


def test_known_answer_learning_journey(ctx):
    """docs/examples/learning-journey/expected-stdout.txt:11-22: inputs [1, 3], weight 0,
    targets [2, 6], summed squared error: objective 40, gradient -40, one step of lr 0.05 gives
    weight 2.0 and predictions [2.0, 6.0]."""
    sess = _scalar_session(ctx, 0.0, Sgd(0.05), reduction="sum")
    sess2 = HipTrainingSession.open(ctx, MlpSpec([Dense(1, 1, None, bias=False)], "mse", "sum"),
                                    [np.zeros((1, 1), np.float32)], [None], Sgd(0.05), 2)
    step = sess2.run(np.array([[1.0], [3.0]]), np.array([[2.0], [6.0]]))
    assert step.objective == 40.0
    assert sess2.state().weights[0][0, 0] == 2.0
    sess.close()
    sess2.close()


def test_non_finite_update_commits_nothing(ctx):
    """A non-finite candidate raises ArithmeticError and leaves parameters, slots and the step
    counter unchanged (TrainingParameter.java:488-525, TrainingSession.java:1151-1170)."""
    spec = MlpSpec.chain([4, 8, 1], hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 8)
    x = np.ones((8, 4), np.float32)
    sess.run(x, np.zeros((8, 1), np.float32))
    before = sess.state()
    with pytest.raises(HipArithmeticError):
        sess.run(x, np.full((8, 1), 3e38, np.float32))
    after = sess.state()
    assert after.optimizer_steps == before.optimizer_steps == 1
    for a, b in zip(before.weights + before.biases + before.first, after.weights + after.biases + after.first):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    sess.run(x, np.zeros((8, 1), np.float32))  # the session stays usable
    assert sess.optimizer_steps == 2
    sess.close()


def test_out_of_range_label_rejected_without_update(ctx):
    spec = MlpSpec.chain([8, 16, 5], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), 4)
    x = np.ones((4, 8), np.float32)
    before = sess.state()
    with pytest.raises(HipIndexError):
        sess.run(x, np.array([0, 1, 5, 2], np.int64))
    after = sess.state()
    assert after.optimizer_steps == 0
    for a, b in zip(before.weights, after.weights):
        assert np.array_equal(a, b)


def test_state_restore_replays_bit_exactly(ctx):
    spec = MlpSpec.chain([16, 32, 1], hidden="sigmoid", loss="mse")
    Ws, bs = init_parameters(spec, 5, "xavier_uniform")
    x, y = _c1_data()
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-2), 256)
    sess.run(x, y)
    snap = sess.state()
    sess.run(x, y)
    second = sess.state()
    sess.restore(snap)
    sess.run(x, y)
    again = sess.state()
    assert again.optimizer_steps == second.optimizer_steps
    for a, b in zip(second.weights + second.first + second.second, again.weights + again.first + again.second):
        assert np.array_equal(a, b)
    sess.close()


@needs_two_streams
def test_failed_two_stream_steps_leave_no_trace(ctx):
    """A classifier step whose program runs on two streams (replayed graph; the step commit is
    performed by the run's last launch) fails on an out-of-range label, then succeeds; two such
    rounds leave exactly the state of a session that only ran the two clean steps."""
    spec = MlpSpec.chain([64, 128, 128, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 3, "he_normal")
    rng = np.random.default_rng(11)
    x = rng.uniform(0, 1, (256, 64)).astype(np.float32)
    good = rng.integers(0, 10, 256).astype(np.int64)
    bad = good.copy()
    bad[200] = 10
    a = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), 256)
    a.program.set_concurrent(True)  # a program this small runs on one stream by default
    assert a.program.side_steps() > 0
    for _ in range(2):
        with pytest.raises(HipIndexError):
            a.run(x, bad)
        a.run(x, good)
    b = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), 256)
    b.run(x, good)
    b.run(x, good)
    sa, sb = a.state(), b.state()
    assert sa.optimizer_steps == sb.optimizer_steps == 2
    for p, q in zip(sa.weights + sa.biases + sa.first + sa.second,
                    sb.weights + sb.biases + sb.first + sb.second):
        assert np.array_equal(p.view(np.uint32), q.view(np.uint32))
    assert a.objective().view(np.uint32) == b.objective().view(np.uint32)
    a.close()
    b.close()


@needs_fold
def test_failure_of_the_folded_bias_update_alone_commits_nothing(ctx):
    """Zero inputs and zero biases make every weight gradient exactly zero (the hidden ReLU is
    off, its gradient masked to zero), while the output bias gradient under MSE SUM, the column
    sum of 32 rows of 2 * (0 - 1.5e38), overflows: only the bias update, which the run's last
    launch performs (a program this small folds it), flags the status word. The run raises
    ArithmeticError and commits nothing -- the last launch reads the word after its own update
    -- in the folded form and in the profiled form that launches the update on its own."""
    from synaptik_amd.native import program_plan
    spec = MlpSpec(MlpSpec.chain([4, 8, 1], hidden="relu").layers, "mse", "sum")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    pb, _ = lower_training_step(spec, 32, Sgd(0.1))
    assert program_plan(pb.image())[2][1] >= 0  # the bias update is folded
    x = np.zeros((32, 4), np.float32)
    bad = np.full((32, 1), 1.5e38, np.float32)
    for profiled in (False, True):
        sess = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1), 32)
        sess.program.set_profiling(profiled)
        before = sess.state()
        with pytest.raises(HipArithmeticError):
            sess.run(x, bad)
        after = sess.state()
        assert after.optimizer_steps == before.optimizer_steps == 0, profiled
        for a, b in zip(before.weights + before.biases, after.weights + after.biases):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), profiled
        sess.run(x, np.zeros((32, 1), np.float32))
        assert sess.optimizer_steps == 1
        sess.close()


def test_folded_bias_update_matches_its_own_launch(ctx):
    """The C1 network's bias update runs in the run's last launch; profiled runs launch it on its
    own. Five steps of each give bit-identical objectives, parameters and counters."""
    spec = MlpSpec.chain([16, 64, 1], hidden="tanh", loss="mse")
    Ws, bs = init_parameters(spec, 0, "builder")
    rng = np.random.default_rng(2)
    a = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.01), 256)
    b = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.01), 256)
    b.program.set_profiling(True)
    for step in range(5):
        x = rng.standard_normal((256, 16)).astype(np.float32)
        y = rng.standard_normal((256, 1)).astype(np.float32)
        oa, ob = a.run(x, y).objective, b.run(x, y).objective
        assert np.float32(oa).view(np.uint32) == np.float32(ob).view(np.uint32), step
    sa, sb = a.state(), b.state()
    assert sa.optimizer_steps == sb.optimizer_steps == 5
    for u, v in zip(sa.weights + sa.biases, sb.weights + sb.biases):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
    a.close()
    b.close()


def test_c3_classifier_from_builder_seeded_he_normal_weights(ctx):
    """The C3 network with the weights bench.py trains: Linear's kaimingReluNormal policy over one
    L64X128MixRandom per ModelBuilder step (nextGaussian per weight, row-major). Four Adam steps
    at batch 128 against the oracle from the same initial bytes."""
    batch = 128
    spec = MlpSpec.chain([784, 1024, 1024, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 0, "builder_he_normal")
    for W, l in zip(Ws, spec.layers):  # He-normal: standard deviation sqrt(2 / fan_in)
        assert abs(float(W.std()) / np.sqrt(2.0 / l.fan_in) - 1.0) < 0.05
    rng = np.random.default_rng(3)
    x = rng.uniform(0, 1, size=(batch, 784)).astype(np.float32)
    labels = rng.integers(0, 10, size=batch).astype(np.int64)
    ref = oracle.OracleMLP(Ws, bs, ["relu", "relu", None], "ce",
                           dict(kind="adam", lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8))
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3, 0.9, 0.999, 1e-8), batch)
    got = [sess.run(x, labels).objective for _ in range(4)]
    want = [float(ref.step(x, labels)) for _ in range(4)]
    np.testing.assert_allclose(got, want, rtol=1e-4)
    sess.close()
