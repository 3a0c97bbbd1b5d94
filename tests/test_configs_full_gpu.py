"""The benchmark configurations at their full sizes on the GPU.

C3 (784->1024->1024->10 ReLU, softmax-CE, Adam(1e-3, 0.9, 0.999, 1e-8), batch 1024) is compared
with the oracle for 3 steps (the oracle's cost bounds the count). C4 (MLP-4096, batch 4096) is too
large for the oracle, so it is checked through size-independent properties: the first objective
equals a float64 forward pass, reductions are deterministic (a replay from a restored state is
bit-identical), and the objective stays finite while training.
"""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.training import Adam, HipTrainingSession, MlpSpec, Sgd, init_parameters

pytestmark = pytest.mark.gpu


def test_c3_full_batch_three_steps_against_oracle(ctx):
    spec = MlpSpec.chain([784, 1024, 1024, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    rng = np.random.default_rng(1)
    x = rng.uniform(0, 1, (1024, 784)).astype(np.float32)
    y = rng.integers(0, 10, 1024).astype(np.int64)
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3, 0.9, 0.999, 1e-8), 1024)
    ref = oracle.OracleMLP(Ws, bs, ["relu", "relu", None], "ce",
                           dict(kind="adam", lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8))
    got, want = [], []
    for _ in range(3):
        got.append(sess.run(x, y).objective)
        want.append(float(ref.step(x, y)))
    np.testing.assert_allclose(got, want, rtol=1e-4)
    st = sess.state()
    for a, b in zip(st.weights + st.biases, ref.W + ref.b):
        assert np.linalg.norm(a.reshape(b.shape) - b) / np.linalg.norm(b) < 1e-5
    sess.close()


def test_c4_full_size_properties(ctx):
    W = 4096
    spec = MlpSpec.chain([W] * 6, hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    rng = np.random.default_rng(1)
    x = rng.standard_normal((W, W), dtype=np.float32)
    y = rng.standard_normal((W, W), dtype=np.float32)
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.01, momentum=0.9), W)
    bx, by = ctx.upload(x), ctx.upload(y)
    # first objective vs a float64 forward pass of the same network
    h = x.astype(np.float64)
    for i, w in enumerate(Ws):
        h = h @ w.T.astype(np.float64)
        if i < 4:
            h = np.maximum(h, 0.0)
    want = float(np.mean((h - y) ** 2))
    sess.run_resident(bx, by)
    first = float(sess.objective())
    assert abs(first - want) <= 1e-4 * want
    snap = sess.state()
    objs = []
    for _ in range(3):
        sess.run_resident(bx, by)
        objs.append(float(sess.objective()))
    after = sess.state()
    # replay from the snapshot: bit-identical objectives and parameters (deterministic kernels)
    sess.restore(snap)
    replay = []
    for _ in range(3):
        sess.run_resident(bx, by)
        replay.append(float(sess.objective()))
    again = sess.state()
    assert replay == objs
    assert again.optimizer_steps == after.optimizer_steps == 4
    for a, b in zip(after.weights + after.biases + after.first, again.weights + again.biases + again.first):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert all(np.isfinite(o) for o in objs) and objs[-1] < first
    sess.close()
