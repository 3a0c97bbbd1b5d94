"""SPI mirror on the GPU: compiler-shaped partitions executed through preparer -> finalizer ->
prepared executable -> bound invocation, checked against the oracle."""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.backend import (HipPartitionFinalizer, HipPartitionPreparer, Node, Partition,
                                  TensorDescriptor as T)
from tests.partitions import f32, mlp_train_partition, softmax_ce_partition

pytestmark = pytest.mark.gpu


def prepare(ctx, part):
    return HipPartitionFinalizer(ctx).finalize_partition(HipPartitionPreparer().analyze(part))


@pytest.mark.parametrize("dims", [(16, 8, 12, 4), (256, 64, 96, 10), (1024, 512, 768, 256)])
def test_mlp_training_partition_matches_oracle(ctx, dims):
    B, I, H, O = dims
    rng = np.random.default_rng(B)
    x = rng.standard_normal((B, I)).astype(np.float32)
    W1 = (rng.standard_normal((H, I)) * np.sqrt(2 / I)).astype(np.float32)
    b1 = (rng.standard_normal(H) * 0.1).astype(np.float32)
    W2 = (rng.standard_normal((O, H)) * np.sqrt(2 / H)).astype(np.float32)
    b2 = (rng.standard_normal(O) * 0.1).astype(np.float32)
    t = rng.standard_normal((B, O)).astype(np.float32)
    exe = prepare(ctx, mlp_train_partition(B, I, H, O))
    got = exe.run_values({"x": x, "W1": W1, "b1": b1, "W2": W2, "b2": b2, "t": t})
    ref = oracle.OracleMLP([W1, W2], [b1, b2], ["relu", None], "mse", dict(kind="sgd", lr=0.1))
    loss, gW, gb, xs = ref.gradients(x, t)
    # the reference sums the MSE sequentially in binary32; the GPU sum is (nearly) exactly rounded
    exact = np.mean((xs[-1].astype(np.float64) - t) ** 2)
    assert abs(got["L"] - exact) <= 1e-6 * exact
    assert abs(got["L"] - loss) <= 1e-4 * abs(loss)
    np.testing.assert_allclose(got["P"], xs[-1], rtol=1e-5, atol=1e-5)
    for name, want in [("dW2", gW[1]), ("db2", gb[1])]:
        rel = np.linalg.norm(got[name] - want) / np.linalg.norm(want)
        assert rel < 1e-5, (name, rel)
    # The ReLU mask is a predicate on Z1b: an element within rounding of zero may fall on the
    # other side in the GPU's reduction order. Bound those flips, then check the first layer's
    # gradients against the oracle's backward driven by the GPU's own mask.
    z_ref = oracle.matmul(x, W1, trans_b=True) + b1
    mask = got["Z1b"] > 0
    assert np.mean(mask != (z_ref > 0)) < 1e-4
    dP = oracle.mse_grad(xs[-1], t)
    dZ1 = np.where(mask, oracle.matmul(dP, W2), np.float32(0)).astype(np.float32)
    for name, want in [("dW1", oracle.matmul(dZ1, x, trans_a=True)), ("db1", oracle.colsum(dZ1))]:
        rel = np.linalg.norm(got[name] - want) / np.linalg.norm(want)
        assert rel < 1e-5, (name, rel)
    exe.close()


def test_softmax_ce_partition_matches_oracle(ctx):
    R, C = 300, 10
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((R, C)) * 3).astype(np.float32)
    g = rng.standard_normal((R, C)).astype(np.float32)
    labels = rng.integers(0, C, R).astype(np.int64)
    exe = prepare(ctx, softmax_ce_partition(R, C))
    got = exe.run_values({"x": x, "g": g, "labels": labels})
    p = oracle.softmax_rows(x)
    np.testing.assert_allclose(got["p"], p, rtol=2e-6, atol=1e-30)
    np.testing.assert_allclose(got["dx"], oracle.softmax_grad_rows(p, g), rtol=1e-5, atol=1e-7)
    lse = oracle.logsumexp_rows(x)
    np.testing.assert_allclose(got["lse"], lse, rtol=1e-6)
    assert abs(got["m"] - oracle.exact_mean(lse)) <= 1e-6 * abs(got["m"])
    ce = oracle.index_ce_mean(x, labels)
    assert abs(got["ce"] - ce) <= 1e-5 * abs(ce)
    np.testing.assert_allclose(got["lsm"], oracle.softmax_rows(x, log=True), rtol=1e-6, atol=2e-6)
    exe.close()


def test_prepared_executable_is_reusable_and_rejects_foreign_buffers(ctx):
    part = Partition({"x": f32(64, 32), "y": f32(64, 32), "z": f32(64, 32)},
                     [Node("TANH", ["x"], "y"), Node("MUL", ["y", "y"], "z")], ["x"], ["z"])
    exe = prepare(ctx, part)
    rng = np.random.default_rng(2)
    for _ in range(3):
        x = rng.standard_normal((64, 32)).astype(np.float32)
        out = exe.run_values({"x": x})["z"]
        y = oracle.activation("tanh", x)
        assert np.array_equal(out, y * y)
    with pytest.raises(ValueError):
        exe.bind({"x": np.zeros(4)})
    exe.close()


_GOLDEN = __import__("json").loads(
    (__import__("pathlib").Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def _golden_val(v):
    if isinstance(v, str):
        return {"inf": np.inf, "-inf": -np.inf, "nan": np.nan, "-0": -0.0}[v]
    return float(v)


@pytest.mark.parametrize("case", _GOLDEN["softmax_backward"],
                         ids=lambda c: f"{'log' if c['log'] else 'softmax'}-{c['case']}")
def test_softmax_backward_graph_reference_known_answers(ctx, case):
    """The softmax / log-softmax gradient graphs as ReductionGradientRules.java:84-90 emits them
    (MUL, keepdims SUM, SUB [, EXP]) through the SPI, bit for bit against
    CpuSoftmaxBackwardConformanceTest's cases (saved outputs y and seeds g given; NaN payloads
    free), non-finite operands included."""
    y = np.array([_golden_val(v) for v in case["y"]], np.float32).reshape(2, 3)
    g = np.array([_golden_val(v) for v in case["g"]], np.float32).reshape(2, 3)
    if case["log"]:
        v = {"y": f32(2, 3), "g": f32(2, 3), "e": f32(2, 3), "s": f32(2, 1), "es": f32(2, 3),
             "dx": f32(2, 3)}
        n = [Node("EXP", ["y"], "e"),
             Node("SUM", ["g"], "s", {"axes": (1,), "keepdims": True}),
             Node("MUL", ["e", "s"], "es"),
             Node("SUB", ["g", "es"], "dx")]
    else:
        v = {"y": f32(2, 3), "g": f32(2, 3), "gy": f32(2, 3), "s": f32(2, 1), "gs": f32(2, 3),
             "dx": f32(2, 3)}
        n = [Node("MUL", ["g", "y"], "gy"),
             Node("SUM", ["gy"], "s", {"axes": (1,), "keepdims": True}),
             Node("SUB", ["g", "s"], "gs"),
             Node("MUL", ["y", "gs"], "dx")]
    exe = prepare(ctx, Partition(v, n, ["y", "g"], ["dx"]))
    got = np.asarray(exe.run_values({"y": y, "g": g})["dx"], np.float32).ravel()
    exe.close()
    for i, w in enumerate(case["expected_bits"]):
        if w is None:
            assert np.isnan(got[i]), (i, got[i])
        else:
            assert int(got[i:i + 1].view(np.uint32)[0]) == w, (i, got[i])
