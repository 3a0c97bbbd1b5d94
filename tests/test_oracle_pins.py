"""Pins the CPU oracle before it is trusted as the parity checker.

Each function of the restatement is checked against something that does not retype its formula:
the reference's own known answers (tests/golden/reference_known_answers.json), exact rational
arithmetic (fractions.Fraction with an independent round-to-binary32), pure-Python brute force on
tiny inputs, float64 numpy / torch autograd as independent mathematics, and closed forms.
"""
import json
import math
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
FMAX = float(np.finfo(np.float32).max)


def _val(v):
    if isinstance(v, str):
        return {"max": FMAX, "-max": -FMAX, "inf": math.inf, "-inf": -math.inf, "nan": math.nan,
                "-0": -0.0}[v]
    return float(v)


def f32_of_fraction(q: Fraction) -> np.float32:
    """Round an exact rational to binary32, ties to even, with subnormals (independent of C)."""
    if q == 0:
        return np.float32(0.0)
    neg = q < 0
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, -126)  # subnormal range shares the 2^-149 quantum
    quantum = Fraction(2) ** (e - 23)
    m = q / quantum
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = fl * quantum
    if val > Fraction(FMAX):
        r = np.float32(np.inf)
    else:
        r = np.float32(float(val))
    return -r if neg else r


def bits(x) -> int:
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


# ---- MATMUL ----
def test_matmul_brute_force_sequential_no_fma():
    rng = np.random.default_rng(1)
    A = rng.standard_normal((3, 5)).astype(np.float32)
    B = rng.standard_normal((5, 4)).astype(np.float32)
    C = oracle.matmul(A, B)
    for i in range(3):
        for j in range(4):
            s = np.float32(0.0)
            for k in range(5):
                s = np.float32(s + np.float32(A[i, k] * B[k, j]))
            assert bits(C[i, j]) == bits(s)


def test_matmul_integer_operands_exact():
    rng = np.random.default_rng(2)
    A = rng.integers(-3, 4, (33, 70)).astype(np.float32)
    B = rng.integers(-3, 4, (70, 21)).astype(np.float32)
    assert np.array_equal(oracle.matmul(A, B), (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32))
    assert np.array_equal(oracle.matmul(A.T.copy(), B, trans_a=True), oracle.matmul(A, B))
    assert np.array_equal(oracle.matmul(A, B.T.copy(), trans_b=True), oracle.matmul(A, B))


def test_matmul_error_bound_against_float64():
    rng = np.random.default_rng(3)
    K = 512
    A = rng.standard_normal((40, K)).astype(np.float32)
    B = rng.standard_normal((K, 30)).astype(np.float32)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    bound = K * 2.0 ** -24 / (1 - K * 2.0 ** -24) * (np.abs(A).astype(np.float64) @ np.abs(B))
    assert (np.abs(oracle.matmul(A, B) - exact) <= bound).all()


@pytest.mark.parametrize("case", GOLDEN["matmul_special"], ids=lambda c: c["case"])
def test_matmul_special_values(case):
    m, n, k = case["m"], case["n"], case["k"]
    A = np.array([_val(v) for v in case["a"]], np.float32).reshape(m, k)
    B = np.array([_val(v) for v in case["b"]], np.float32).reshape(k, n)
    C = oracle.matmul(A, B)
    assert [bits(v) for v in C.ravel()] == case["expected_bits"]


# ---- exact SUM / MEAN / quotient ----
@pytest.mark.parametrize("seed", range(5))
def test_exact_sum_and_mean_match_rational_arithmetic(seed):
    rng = np.random.default_rng(seed)
    n = 1000
    x = (rng.standard_normal(n) * np.exp(rng.uniform(-30, 30, n))).astype(np.float32)
    exact = sum(Fraction(float(v)) for v in x)
    assert bits(oracle.exact_sum(x)) == bits(f32_of_fraction(exact))
    assert bits(oracle.exact_mean(x)) == bits(f32_of_fraction(exact / n))


def test_exact_sum_cancellation_and_subnormals():
    assert oracle.exact_sum(np.array([1e30, 1, -1e30], np.float32)) == 1.0
    tiny = np.float32(1.4e-45)
    assert bits(oracle.exact_sum(np.array([tiny, tiny, tiny], np.float32))) == 3
    assert np.isnan(oracle.exact_sum(np.array([np.inf, -np.inf], np.float32)))
    assert oracle.exact_sum(np.array([FMAX, FMAX], np.float32)) == np.inf
    assert bits(oracle.exact_sum(np.array([-0.0, -0.0], np.float32))) == 0  # exact zero is +0


def _bits32(v) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


@pytest.mark.parametrize("xs,want", [
    ([], -math.inf),                       # empty domain: -infinity (AggregateReductionKind.java:133)
    ([-0.0, 0.0], 0.0),                    # +0 is selected over -0, in either order
    ([0.0, -0.0], 0.0),
    ([-0.0, -0.0], -0.0),
    ([-0.0], -0.0),                        # a singleton keeps its sign
    ([-1e-45, -0.0, -3.0], -0.0),
    ([1e-45, 2e-45, -1.0], 2e-45),         # subnormals compared as stored, never flushed
    ([-2e-45, -1e-45], -1e-45),
    ([-math.inf, -math.inf], -math.inf),
    ([1.0, math.inf, 2.0], math.inf),
    ([-FMAX, -math.inf], -FMAX),
], ids=lambda v: str(v))
def test_max_special_values(xs, want):
    got = oracle.max_reduce(np.array(xs, np.float32))
    assert _bits32(got) == _bits32(want)


def test_max_propagates_nan_anywhere():
    for pos in range(5):
        x = np.array([1.0, -0.0, math.inf, 3.0, 0.0], np.float32)
        x[pos] = math.nan
        assert math.isnan(oracle.max_reduce(x))
    assert math.isnan(oracle.max_reduce(np.array([math.nan, math.inf], np.float32)))


def test_max_is_numpy_selection_without_zeros_or_nan():
    rng = np.random.default_rng(9)
    X = (rng.standard_normal((40, 1001)) * 100).astype(np.float32)
    X[X == 0] = 1.0
    assert np.array_equal(oracle.max_rows(X).view(np.uint32), X.max(axis=1).view(np.uint32))
    assert _bits32(oracle.max_reduce(X)) == _bits32(X.max())


def test_exact_quotient_is_rounded_once():
    for v, n in [(1.0, 3), (2.0, 7), (1e-38, 3), (123456.789, 4096 * 4096)]:
        q = oracle.exact_quotient(v, n)
        assert bits(q) == bits(f32_of_fraction(Fraction(float(np.float32(v))) / n))


def test_colsum_is_exact_per_column():
    rng = np.random.default_rng(9)
    X = (rng.standard_normal((257, 5)) * 1e4).astype(np.float32)
    got = oracle.colsum(X)
    for c in range(5):
        assert bits(got[c]) == bits(f32_of_fraction(sum(Fraction(float(v)) for v in X[:, c])))


# ---- activations ----
def test_activations_match_binary64_math():
    x = np.linspace(-20, 20, 4001).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf], np.float32)])
    d = x.astype(np.float64)
    assert np.array_equal(oracle.activation("tanh", x), np.tanh(d).astype(np.float32))
    sig = np.where(d >= 0, 1 / (1 + np.exp(-np.abs(d))), np.exp(-np.abs(d)) / (1 + np.exp(-np.abs(d))))
    np.testing.assert_array_max_ulp(oracle.activation("sigmoid", x), sig.astype(np.float32), maxulp=1)
    r = oracle.activation("relu", np.array([-1, -0.0, 0.0, 2, np.nan], np.float32))
    assert [bits(v) for v in r[:4]] == [0, 0, 0, bits(2.0)] and np.isnan(r[4])


def test_activation_gradients_closed_forms():
    y = np.array([0.5, -0.25, 0.0, 0.9], np.float32)
    g = np.array([2.0, 4.0, 1.0, -1.0], np.float32)
    assert list(oracle.activation_grad("tanh", g, y)[:3]) == [1.5, 3.75, 1.0]
    assert oracle.activation_grad("sigmoid", g, y)[0] == 0.5
    assert list(oracle.activation_grad("relu", g, y)) == [2.0, 0.0, 0.0, -1.0]


# ---- softmax / LSE ----
@pytest.mark.parametrize("case", GOLDEN["softmax_rows"], ids=lambda c: c["source"][-30:])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_reference_known_answers(case, log):
    x = np.array([[_val(v) for v in case["x"]]], np.float32)
    got = oracle.softmax_rows(x, log=log)[0]
    want = [_val(v) for v in case["log_softmax" if log else "softmax"]]
    for g, w in zip(got, want):
        if math.isnan(w):
            assert math.isnan(g)
        elif math.isinf(w) or case["tolerance"] == 0.0:
            assert g == w
        else:
            assert abs(g - w) <= case["tolerance"]


def _bits_match(got, want_bits):
    for i, (g, w) in enumerate(zip(np.asarray(got, np.float32).ravel(), want_bits)):
        if w is None:
            assert math.isnan(g), i
        else:
            assert int(np.array([g], np.float32).view(np.uint32)[0]) == w, (i, g)


@pytest.mark.parametrize("case", [c for c in GOLDEN["softmax_backward"] if not c["log"]],
                         ids=lambda c: c["case"])
def test_softmax_backward_reference_known_answers(case):
    """CpuSoftmaxBackwardConformanceTest's softmax rows, bit for bit (NaN payloads free)."""
    y = np.array([_val(v) for v in case["y"]], np.float32).reshape(2, 3)
    g = np.array([_val(v) for v in case["g"]], np.float32).reshape(2, 3)
    with np.errstate(all="ignore"):
        _bits_match(oracle.softmax_grad_rows(y, g), case["expected_bits"])


def test_softmax_against_float64_and_invariants():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((64, 300)) * 2).astype(np.float32)
    x[rng.random(x.shape) < 0.01] = 30.0
    p = oracle.softmax_rows(x)
    d = x.astype(np.float64)
    e = np.exp(d - d.max(1, keepdims=True))
    ref = e / e.sum(1, keepdims=True)
    np.testing.assert_allclose(p, ref, rtol=2e-6, atol=1e-12)
    np.testing.assert_allclose(p.astype(np.float64).sum(1), 1.0, rtol=1e-5)
    lp = oracle.softmax_rows(x, log=True)
    lse = oracle.logsumexp_rows(x)
    np.testing.assert_allclose(lp, x - lse[:, None], rtol=0, atol=5e-5)
    ref_lse = d.max(1) + np.log(np.exp(d - d.max(1, keepdims=True)).sum(1))
    np.testing.assert_allclose(lse, ref_lse, rtol=1e-6)


def test_logsumexp_special_rows():
    x = np.array([[-np.inf, -np.inf], [np.inf, 1.0], [np.nan, 1.0], [0.0, 0.0]], np.float32)
    l = oracle.logsumexp_rows(x)
    assert l[0] == -np.inf and l[1] == np.inf and np.isnan(l[2])
    assert abs(l[3] - math.log(2)) < 1e-7


def test_softmax_and_lse_gradients_against_torch_autograd():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8, 50)).astype(np.float32)
    g = rng.standard_normal((8, 50)).astype(np.float32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    torch.softmax(xt, 1).backward(torch.tensor(g, dtype=torch.float64))
    got = oracle.softmax_grad_rows(oracle.softmax_rows(x), g)
    np.testing.assert_allclose(got, xt.grad.numpy(), rtol=1e-4, atol=1e-6)
    xt2 = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    gl = rng.standard_normal(8).astype(np.float32)
    torch.logsumexp(xt2, 1).backward(torch.tensor(gl, dtype=torch.float64))
    got2 = oracle.logsumexp_grad_rows(x, oracle.logsumexp_rows(x), gl)
    np.testing.assert_allclose(got2, xt2.grad.numpy(), rtol=1e-5, atol=1e-7)


# ---- losses ----
def test_mse_closed_forms_and_exact_quotient():
    p = np.full(7, 3.0, np.float32)
    t = np.full(7, 1.0, np.float32)
    assert oracle.mse_mean(p, t) == 4.0
    assert oracle.mse_sum(p, t) == 28.0
    np.testing.assert_array_equal(oracle.mse_grad(p, t), np.full(7, np.float32(4.0) * np.float32(1 / np.float32(7)), np.float32))
    q = np.array([1.0, 0.0, 0.0], np.float32)
    assert bits(oracle.mse_mean(q, np.zeros(3, np.float32))) == bits(f32_of_fraction(Fraction(1, 3)))


def test_mse_exact_reduction_against_rationals_and_sequential_saturation():
    """mse_mean_exact is the contract's exactly rounded mean of the binary32 squares (Fraction
    arithmetic); the reference CPU kernels' sequential binary32 sum (mse_mean) saturates once
    the running sum reaches 2^24 with unit squares: n = 2^24 + 2^20 ones give a running sum of
    exactly 2^24, so its mean is 2^24 / n, while the exact mean is 1."""
    rng = np.random.default_rng(8)
    p = rng.standard_normal(1001).astype(np.float32)
    t = rng.standard_normal(1001).astype(np.float32)
    sq = [Fraction(float((a - b) * (a - b))) for a, b in zip(p, t)]  # binary32 products
    want = f32_of_fraction(sum(sq, Fraction(0)) / len(sq))
    assert bits(oracle.mse_mean_exact(p, t)) == bits(want)
    n = 2**24 + 2**20
    ones, zeros = np.ones(n, np.float32), np.zeros(n, np.float32)
    assert oracle.mse_mean_exact(ones, zeros) == 1.0
    assert bits(oracle.mse_mean(ones, zeros)) == bits(f32_of_fraction(Fraction(2**24, n)))


def test_index_ce_against_float64_and_bounds():
    rng = np.random.default_rng(6)
    logits = (rng.standard_normal((50, 10)) * 3).astype(np.float32)
    y = rng.integers(0, 10, 50)
    d = logits.astype(np.float64)
    lse = d.max(1) + np.log(np.exp(d - d.max(1, keepdims=True)).sum(1))
    ref = float(np.mean(lse - d[np.arange(50), y]))
    assert abs(oracle.index_ce_mean(logits, y) - ref) <= 1e-5 * abs(ref)
    with pytest.raises(ValueError):
        oracle.index_ce_mean(logits, np.where(np.arange(50) == 3, 10, y))
    with pytest.raises(ValueError):
        oracle.index_ce_mean(logits, np.where(np.arange(50) == 3, -1, y))
    ign = np.where(np.arange(50) < 5, -100, y)
    ref_ign = float(np.mean((lse - d[np.arange(50), np.clip(ign, 0, 9)])[5:]))
    assert abs(oracle.index_ce_mean(logits, ign, ignore_index=-100) - ref_ign) <= 1e-5 * abs(ref_ign)


def test_index_ce_gradient_against_torch_autograd():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((32, 10)).astype(np.float32)
    y = rng.integers(0, 10, 32)
    lt = torch.tensor(logits, dtype=torch.float64, requires_grad=True)
    torch.nn.functional.cross_entropy(lt, torch.tensor(y)).backward()
    np.testing.assert_allclose(oracle.index_ce_grad(logits, y), lt.grad.numpy(), rtol=1e-5, atol=1e-8)
    ign = np.where(np.arange(32) % 4 == 0, -100, y)
    lt2 = torch.tensor(logits, dtype=torch.float64, requires_grad=True)
    torch.nn.functional.cross_entropy(lt2, torch.tensor(ign), ignore_index=-100).backward()
    np.testing.assert_allclose(oracle.index_ce_grad(logits, ign, ignore_index=-100), lt2.grad.numpy(),
                               rtol=1e-5, atol=1e-8)


# ---- optimizers ----
def test_sgd_reference_known_answers():
    cases = {c["case"]: c for c in GOLDEN["training"]}
    c = cases["scalar SGD"]
    w = np.array([2.0], np.float32)
    for st in c["steps"]:
        err = w * st["x"] - st["t"]
        assert abs(float((err * err)[0]) - st["objective"]) < 1e-6
        g = np.float32(2) * err * np.float32(st["x"])
        w, _ = oracle.sgd_stage(w, g, None, lr=0.1)
        assert abs(float(w[0]) - st["w_after"]) <= c["tolerance"]
    c = cases["SGD momentum"]
    w = np.array([2.0], np.float32)
    m = np.zeros(1, np.float32)
    for i, st in enumerate(c["steps"]):
        g = np.float32(2) * w
        w, m = oracle.sgd_stage(w, g, m, lr=0.1, momentum=0.5, completed_steps=i)
        assert abs(float(w[0]) - st["w_after"]) <= c["tolerance"]
    assert abs(float(m[0]) - 5.2) <= 1e-6


def test_adam_matches_reference_test_oracle():
    """AdamOptimizerTest.Oracle (:525-580), a float64 multi-step formula, vs the float oracle."""
    cfg = GOLDEN["adam_oracle"]["config"]
    for decoupled in (False, True):
        p_ref, first, second = 2.0, 0.0, 0.0
        p = np.array([2.0], np.float32)
        m = np.zeros(1, np.float32)
        v = np.zeros(1, np.float32)
        for step in range(1, 6):
            g_pub = 2.0 * p_ref
            grad = g_pub if decoupled else g_pub + cfg["weight_decay"] * p_ref
            first = 0.5 * first + 0.5 * grad
            second = 0.25 * second + 0.75 * grad * grad
            cf = first / (1 - 0.5 ** step)
            cs = second / (1 - 0.25 ** step)
            base = p_ref * (1 - cfg["lr"] * cfg["weight_decay"]) if decoupled else p_ref
            p_ref = base - cfg["lr"] * cf / (math.sqrt(cs) + cfg["eps"])
            p, m, v = oracle.adam_stage(p, np.float32(2) * p, m, v, lr=cfg["lr"], beta1=cfg["beta1"],
                                        beta2=cfg["beta2"], eps=cfg["eps"],
                                        weight_decay=cfg["weight_decay"], decoupled=decoupled,
                                        completed_steps=step - 1)
            assert abs(float(p[0]) - p_ref) <= 1e-6 * max(1.0, abs(p_ref))


def test_optimizer_stages_reject_non_finite():
    with pytest.raises(ArithmeticError):
        oracle.sgd_stage(np.array([1.0], np.float32), np.array([np.inf], np.float32), None, lr=0.1)
    with pytest.raises(ArithmeticError):
        # momentum overflow: 0.9 * 3e38 + 3e38 is not finite
        oracle.sgd_stage(np.array([1.0], np.float32), np.array([3e38], np.float32),
                         np.array([3e38], np.float32), lr=1.0, momentum=0.9, completed_steps=1)
    with pytest.raises(ArithmeticError):
        oracle.adam_stage(np.array([1.0], np.float32), np.array([np.nan], np.float32),
                          np.zeros(1, np.float32), np.zeros(1, np.float32), lr=0.1, beta1=0.9,
                          beta2=0.999, eps=1e-8)


# ---- composition: MLP gradients vs torch autograd ----
@pytest.mark.parametrize("gemm", ["oracle", "float64"])
@pytest.mark.parametrize("loss,act", [("mse", "tanh"), ("mse", "relu"), ("ce", "relu"), ("mse", "sigmoid")])
def test_mlp_gradients_against_torch_autograd(loss, act, gemm):
    torch = pytest.importorskip("torch")
    from synaptik_amd.training import MlpSpec, init_parameters
    widths = [12, 20, 16, 5 if loss == "ce" else 3]
    spec = MlpSpec.chain(widths, hidden=act, loss=loss)
    Ws, bs = init_parameters(spec, 11, "xavier_uniform")
    bs = [np.random.default_rng(i).standard_normal(b.shape).astype(np.float32) * 0.1 for i, b in enumerate(bs)]
    rng = np.random.default_rng(12)
    x = rng.standard_normal((24, widths[0])).astype(np.float32)
    y = rng.integers(0, widths[-1], 24) if loss == "ce" else rng.standard_normal((24, widths[-1])).astype(np.float32)
    model = oracle.OracleMLP(Ws, bs, [act, act, None], loss, dict(kind="sgd", lr=0.1), gemm=gemm)
    obj, gW, gb, _ = model.gradients(x, y)
    tW = [torch.tensor(w, dtype=torch.float64, requires_grad=True) for w in Ws]
    tb = [torch.tensor(b, dtype=torch.float64, requires_grad=True) for b in bs]
    h = torch.tensor(x, dtype=torch.float64)
    fn = {"tanh": torch.tanh, "relu": torch.relu, "sigmoid": torch.sigmoid}[act]
    for i in range(3):
        h = h @ tW[i].T + tb[i]
        if i < 2:
            h = fn(h)
    if loss == "ce":
        L = torch.nn.functional.cross_entropy(h, torch.tensor(y))
    else:
        L = torch.mean((h - torch.tensor(y, dtype=torch.float64)) ** 2)
    L.backward()
    assert abs(float(obj) - L.item()) <= 1e-5 * abs(L.item())
    for a, t in zip(gW + gb, tW + tb):
        np.testing.assert_allclose(a, t.grad.numpy(), rtol=1e-4, atol=1e-6)


def test_float64_gemm_mode_tracks_the_oracle_gemm_over_steps():
    """The binary64-GEMM composition (used where the scalar GEMM is too slow) follows the
    reference-order composition over several Adam and SGD-momentum steps within the parity
    tolerance, and its integer-operand GEMMs are bit-identical (exact sums)."""
    from synaptik_amd.training import MlpSpec, init_parameters
    spec = MlpSpec.chain([40, 64, 48, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 5, "he_normal")
    rng = np.random.default_rng(6)
    x = rng.uniform(0, 1, (96, 40)).astype(np.float32)
    y = rng.integers(0, 10, 96)
    for opt in (dict(kind="adam", lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8),
                dict(kind="sgd", lr=0.05, momentum=0.9)):
        a = oracle.OracleMLP(Ws, bs, ["relu", "relu", None], "ce", opt)
        b = oracle.OracleMLP(Ws, bs, ["relu", "relu", None], "ce", opt, gemm="float64")
        la = [float(a.step(x, y)) for _ in range(10)]
        lb = [float(b.step(x, y)) for _ in range(10)]
        np.testing.assert_allclose(lb, la, rtol=1e-5)
        for u, v in zip(a.W + a.b, b.W + b.b):
            assert np.linalg.norm(u - v) <= 1e-5 * np.linalg.norm(u)
    A = rng.integers(-3, 4, (33, 70)).astype(np.float32)
    B = rng.integers(-3, 4, (70, 21)).astype(np.float32)
    m = oracle.OracleMLP(Ws, bs, ["relu", "relu", None], "ce", {"kind": "sgd", "lr": 0.1},
                         gemm="float64")
    assert np.array_equal(m._mm(A, B), oracle.matmul(A, B))
    assert np.array_equal(m._mm(A.T.copy(), B, trans_a=True), oracle.matmul(A, B))


@pytest.mark.parametrize("decoupled,decay", [(False, 0.0), (False, 0.01), (True, 0.1)])
def test_adam_apply_is_the_tail_of_adam_stage(decoupled, decay):
    """adam_apply from the moments adam_stage produced gives adam_stage's parameters bit for bit
    (the same tail; adam_stage is pinned by the reference's multi-step Adam oracle)."""
    rng = np.random.default_rng(3)
    p, g, m = (rng.standard_normal(5000).astype(np.float32) for _ in range(3))
    v = np.abs(rng.standard_normal(5000)).astype(np.float32)
    kw = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=decay, decoupled=decoupled)
    for steps in (0, 1, 7, 500):
        pc, mc, vc = oracle.adam_stage(p, g, m, v, completed_steps=steps, **kw)
        got = oracle.adam_apply(p, mc, vc, completed_steps=steps, **kw)
        assert np.array_equal(got.view(np.uint32), pc.view(np.uint32))
