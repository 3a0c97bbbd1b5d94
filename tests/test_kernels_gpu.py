"""Kernel-level parity on the GPU against the oracle (and the reference's known answers).

Elementwise kernels perform the oracle's exact operation sequence and must be bit-identical;
reductions accumulate in binary64 through a fixed tree (the reference uses exact limb sums or
Kahan binary32), so they are checked to 1 binary32 ulp or a stated relative tolerance.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.native import HipArithmeticError, HipIndexError, HipProgram
from synaptik_amd.program import ProgramBuilder
from synaptik_amd.training import lower_dense_layer
from tests.gpu_helpers import run_program

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
FMAX = float(np.finfo(np.float32).max)


def _val(v):
    if isinstance(v, str):
        return {"max": FMAX, "-max": -FMAX, "inf": math.inf, "-inf": -math.inf, "nan": math.nan,
                "-0": -0.0}[v]
    return float(v)


def gpu_softmax(ctx, x, log=False, with_lse=True):
    R, C = x.shape
    pb = ProgramBuilder()
    sx = pb.input(R * C)
    sy = pb.output(R * C)
    sl = pb.output(R) if with_lse else None
    pb.softmax(sx, sy, R, C, lse=sl, log=log)
    outs = run_program(ctx, pb, [x], [sy] + ([sl] if with_lse else []))
    return outs[0].reshape(R, C), (outs[1] if with_lse else None)


# ---- matmul special values (GEMM entry) ----
@pytest.mark.parametrize("case", GOLDEN["matmul_special"], ids=lambda c: c["case"])
def test_gemm_special_values(ctx, case):
    m, n, k = case["m"], case["n"], case["k"]
    A = np.array([_val(v) for v in case["a"]] or [0.0], np.float32)
    B = np.array([_val(v) for v in case["b"]] or [0.0], np.float32)
    pb = ProgramBuilder()
    sa, sb = pb.input(A.size), pb.input(B.size)
    sc = pb.output(m * n)
    pb.gemm(sa, sb, sc, m, n, k, lda=max(k, 1), ldb=max(n, 1))
    (C,) = run_program(ctx, pb, [A, B], [sc])
    assert [int(v) for v in C.view(np.uint32)] == case["expected_bits"]


# ---- pointwise ----
def test_pointwise_chain_with_broadcast_bit_exact(ctx):
    R, C = 300, 257
    rng = np.random.default_rng(0)
    x = rng.standard_normal((R, C)).astype(np.float32)
    g = rng.standard_normal((R, C)).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    pb = ProgramBuilder()
    sx, sg, sb = pb.input(R * C), pb.input(R * C), pb.input(C)
    o1, o2 = pb.output(R * C), pb.output(R * C)
    code = [("load", 0, 0, 0, 0, 0.0), ("load", 1, 2, 0, 0, 0.0), ("add", 2, 0, 1, 0, 0.0),
            ("tanh", 3, 2, 0, 0, 0.0), ("store", 0, 3, 0, 0, 0.0), ("load", 4, 1, 0, 0, 0.0),
            ("tanh_grad", 5, 3, 4, 0, 0.0), ("const", 6, 0, 0, 0, 0.5), ("mul", 5, 5, 6, 0, 0.0),
            ("store", 1, 5, 0, 0, 0.0)]
    pb.pointwise(R, C, [sx, sg, sb], [o1, o2], code, modes=["full", "full", "row"])
    y, d = run_program(ctx, pb, [x, g, b], [o1, o2])
    z = (x + b[None, :]).astype(np.float32)
    ry = oracle.activation("tanh", z)
    rd = oracle.activation_grad("tanh", g, ry) * np.float32(0.5)
    assert np.array_equal(y.reshape(R, C), ry)
    assert np.array_equal(d.reshape(R, C), rd)


@pytest.mark.parametrize("act", ["relu", "sigmoid"])
def test_pointwise_activation_forward_and_grad(ctx, act):
    n = 10007
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(n) * 5).astype(np.float32)
    x[:4] = [0.0, -0.0, np.inf, -np.inf]
    g = rng.standard_normal(n).astype(np.float32)
    pb = ProgramBuilder()
    sx, sg = pb.input(n), pb.input(n)
    o1, o2 = pb.output(n), pb.output(n)
    pb.pointwise(1, n, [sx, sg], [o1, o2],
                 [("load", 0, 0, 0, 0, 0.0), (act, 1, 0, 0, 0, 0.0), ("store", 0, 1, 0, 0, 0.0),
                  ("load", 2, 1, 0, 0, 0.0), (act + "_grad", 3, 1, 2, 0, 0.0), ("store", 1, 3, 0, 0, 0.0)])
    y, d = run_program(ctx, pb, [x, g], [o1, o2])
    ry = oracle.activation(act, x)
    assert np.array_equal(y.view(np.uint32), ry.view(np.uint32))
    assert np.array_equal(d, oracle.activation_grad(act, g, ry))


# ---- reductions ----
@pytest.mark.parametrize("R,N", [(1, 1), (4096, 4096), (1000, 10), (8192, 1024), (3, 70000), (517, 12), (1025, 1284), (32768, 256), (20000, 100), (32769, 3)])
def test_colsum_against_exact_oracle(ctx, R, N):
    rng = np.random.default_rng(R + N)
    x = rng.standard_normal((R, N)).astype(np.float32)
    pb = ProgramBuilder()
    sx = pb.input(R * N)
    so = pb.output(N)
    pb.colsum(sx, so, R, N)
    (got,) = run_program(ctx, pb, [x], [so])
    np.testing.assert_array_max_ulp(got, oracle.colsum(x), maxulp=1)


@pytest.mark.parametrize("kind", ["sum", "mean", "max", "lse"])
def test_row_reduce(ctx, kind):
    R, C = 257, 3001
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((R, C)) * 3).astype(np.float32)
    x[5, 7] = np.nan
    x[6, :] = -np.inf
    x[7, 3] = np.inf
    pb = ProgramBuilder()
    sx, so = pb.input(R * C), pb.output(R)
    pb.row_reduce(sx, so, R, C, kind)
    (got,) = run_program(ctx, pb, [x], [so])
    if kind == "sum":
        want = np.array([oracle.exact_sum(r) for r in x], np.float32)
    elif kind == "mean":
        want = np.array([oracle.exact_mean(r) for r in x], np.float32)
    elif kind == "max":
        want = oracle.max_rows(x)
    else:
        want = oracle.logsumexp_rows(x)
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)])
    if kind == "max":  # a selection: bit-exact
        assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    elif kind in ("sum", "mean"):
        np.testing.assert_array_max_ulp(got[fin], want[fin], maxulp=1)
    else:
        np.testing.assert_allclose(got[fin], want[fin], rtol=1e-6)


@pytest.mark.parametrize("kind", ["sum", "mean", "max"])
def test_reduce_all(ctx, kind):
    n = 3_000_001
    rng = np.random.default_rng(4)
    x = rng.standard_normal(n).astype(np.float32)
    pb = ProgramBuilder()
    sx, so = pb.input(n), pb.output(1)
    pb.reduce_all(sx, so, n, kind)
    (got,) = run_program(ctx, pb, [x], [so])
    want = {"sum": oracle.exact_sum, "mean": oracle.exact_mean, "max": oracle.max_reduce}[kind](x)
    if kind == "max":
        assert got.view(np.uint32)[0] == np.array([want], np.float32).view(np.uint32)[0]
    else:
        np.testing.assert_array_max_ulp(got, np.array([want], np.float32), maxulp=1)


def _max_special_rows(C):
    """Rows whose MAX exercises Math.max's rules: signed-zero mixes (expect +0 when any +0),
    all -0, NaN at the first / middle / last position, subnormal-only, -inf-only and an
    infinity with NaN; every other row is random."""
    rng = np.random.default_rng(C)
    rows = []
    z = np.where(rng.random(C) < 0.5, np.float32(-0.0), np.float32(0.0))
    z[rng.integers(C)] = 0.0
    rows.append(z)                                                   # -0/+0 mix -> +0
    rows.append(np.full(C, -0.0, np.float32))                        # all -0 -> -0
    neg = -np.abs(rng.standard_normal(C)).astype(np.float32) - 1.0
    nz = neg.copy()
    nz[rng.integers(C)] = -0.0
    rows.append(nz)                                                  # negatives and one -0 -> -0
    for pos in (0, C // 2, C - 1):
        r = rng.standard_normal(C).astype(np.float32)
        r[pos] = np.nan
        rows.append(r)                                               # NaN anywhere -> NaN
    sub = (rng.integers(1, 1 << 20, C).astype(np.uint32)).view(np.float32).copy()
    sub[::3] *= -1
    rows.append(sub)                                                 # subnormals, not flushed
    rows.append(np.full(C, -np.inf, np.float32))
    r = rng.standard_normal(C).astype(np.float32)
    r[1] = np.inf
    r[C - 2] = np.nan
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("C", [5, 64, 3001, 70000])
def test_row_max_math_max_rules_bit_exact(ctx, C):
    x = _max_special_rows(C)
    R = x.shape[0]
    pb = ProgramBuilder()
    sx, so = pb.input(R * C), pb.output(R)
    pb.row_reduce(sx, so, R, C, "max")
    (got,) = run_program(ctx, pb, [x], [so])
    want = oracle.max_rows(x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("n", [1, 255, 256 * 1024 + 3, 3_000_001])
@pytest.mark.parametrize("case", ["zeros-mixed", "zeros-neg", "nan-first", "nan-last",
                                  "nan-middle", "subnormal", "neg-inf"])
def test_reduce_all_max_math_max_rules_bit_exact(ctx, n, case):
    """Whole-tensor MAX: both passes (per-block partials, then the fold over the partials)
    must keep the signed-zero, NaN and subnormal rules."""
    rng = np.random.default_rng(n)
    if case.startswith("zeros"):
        x = np.full(n, -0.0, np.float32)
        if case == "zeros-mixed":
            x[rng.integers(n)] = 0.0   # a single +0 in one block's partition
    elif case.startswith("nan"):
        x = rng.standard_normal(n).astype(np.float32)
        x[{"nan-first": 0, "nan-last": n - 1, "nan-middle": n // 2}[case]] = np.nan
    elif case == "subnormal":
        x = -(rng.integers(1, 1 << 20, n).astype(np.uint32)).view(np.float32)
    else:
        x = np.full(n, -np.inf, np.float32)
    pb = ProgramBuilder()
    sx, so = pb.input(n), pb.output(1)
    pb.reduce_all(sx, so, n, "max")
    (got,) = run_program(ctx, pb, [x], [so])
    want = oracle.max_reduce(x)
    if np.isnan(want):
        assert np.isnan(got[0])
    else:
        assert got.view(np.uint32)[0] == np.array([want], np.float32).view(np.uint32)[0]


# ---- softmax / LSE ----
@pytest.mark.parametrize("case", GOLDEN["softmax_rows"], ids=lambda c: c["source"][-30:])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_reference_known_answers(ctx, case, log):
    x = np.array([[_val(v) for v in case["x"]]], np.float32)
    got, _ = gpu_softmax(ctx, x, log=log)
    want = [_val(v) for v in case["log_softmax" if log else "softmax"]]
    for g, w in zip(got[0], want):
        if math.isnan(w):
            assert math.isnan(g)
        elif math.isinf(w) or case["tolerance"] == 0.0:
            assert g == w
        else:
            assert abs(g - w) <= case["tolerance"]


@pytest.mark.parametrize("C", [10, 1000, 2048, 4096, 5000, 4097])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_rows_against_oracle(ctx, C, log):
    R = 64
    rng = np.random.default_rng(C)
    x = (rng.standard_normal((R, C)) * 2).astype(np.float32)
    x[rng.random(x.shape) < 0.01] = 30.0
    x[3, 1] = -np.inf
    got, lse = gpu_softmax(ctx, x, log=log)
    want = oracle.softmax_rows(x, log=log)
    if log:
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=2e-6)
    else:
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)
    np.testing.assert_allclose(lse, oracle.logsumexp_rows(x), rtol=1e-6)


@pytest.mark.parametrize("C", [10, 4096, 5000])
def test_softmax_backward_against_oracle(ctx, C):
    R = 128
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((R, C)) * 2).astype(np.float32)
    y = oracle.softmax_rows(x)
    g = rng.standard_normal((R, C)).astype(np.float32)
    pb = ProgramBuilder()
    sy, sg, sd = pb.input(R * C), pb.input(R * C), pb.output(R * C)
    pb.softmax_bwd(sy, sg, sd, R, C)
    (d,) = run_program(ctx, pb, [y, g], [sd])
    want = oracle.softmax_grad_rows(y, g)
    np.testing.assert_allclose(d.reshape(R, C), want, rtol=1e-5, atol=1e-7)


def test_lse_backward_against_oracle(ctx):
    R, C = 100, 777
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((R, C)) * 2).astype(np.float32)
    lse = oracle.logsumexp_rows(x)
    g = rng.standard_normal(R).astype(np.float32)
    pb = ProgramBuilder()
    sx, sl, sg, sd = pb.input(R * C), pb.input(R), pb.input(R), pb.output(R * C)
    pb.lse_bwd(sx, sl, sd, R, C, g=sg)
    (d,) = run_program(ctx, pb, [x, lse, g], [sd])
    assert np.array_equal(d.reshape(R, C), oracle.logsumexp_grad_rows(x, lse, g))


# ---- losses ----
@pytest.mark.parametrize("n,reduction", [(1, "mean"), (256, "mean"), (100003, "mean"), (64, "sum")])
def test_mse_against_oracle(ctx, n, reduction):
    rng = np.random.default_rng(n)
    p = rng.standard_normal(n).astype(np.float32)
    t = rng.standard_normal(n).astype(np.float32)
    pb = ProgramBuilder()
    sp, st = pb.input(n), pb.input(n)
    sl, sg = pb.output(1), pb.output(n)
    pb.mse(sp, st, sl, n, grad=sg, reduction=reduction)
    loss, grad = run_program(ctx, pb, [p, t], [sl, sg])
    assert np.array_equal(grad, oracle.mse_grad(p, t, reduction=reduction))
    want = oracle.mse_mean(p, t) if reduction == "mean" else oracle.mse_sum(p, t)
    # the reference sums sequentially in binary32; the GPU's sum is (nearly) exactly rounded
    exact = np.sum((p.astype(np.float64) - t) ** 2) / (n if reduction == "mean" else 1)
    assert abs(loss[0] - exact) <= 1e-6 * abs(exact)
    assert abs(loss[0] - want) <= 1e-4 * abs(want)


@pytest.mark.parametrize("dtype", ["i64", "i32"])
@pytest.mark.parametrize("ignore", [None, -100])
@pytest.mark.parametrize("shape", [(1024, 10), (9000, 10), (300, 100), (4096, 10), (4097, 3)],
                         ids=["c3", "many-rows", "many-classes", "fused-edge", "unfused-edge"])
def test_index_cross_entropy_against_oracle(ctx, dtype, ignore, shape):
    R, C = shape
    rng = np.random.default_rng(9)
    logits = (rng.standard_normal((R, C)) * 3).astype(np.float32)
    y = rng.integers(0, C, R)
    if ignore is not None:
        y[::7] = ignore
    pb = ProgramBuilder()
    sx = pb.input(R * C)
    sy = pb.input(R, dtype)
    sl, sg = pb.output(1), pb.output(R * C)
    pb.index_ce(sx, sy, sl, R, C, grad=sg, ignore_index=ignore)
    loss, grad = run_program(ctx, pb, [logits, y.astype(np.int64 if dtype == "i64" else np.int32)], [sl, sg])
    want = oracle.index_ce_mean(logits, y, ignore_index=ignore)
    assert abs(loss[0] - want) <= 1e-5 * abs(want)
    np.testing.assert_allclose(grad.reshape(R, C), oracle.index_ce_grad(logits, y, ignore_index=ignore),
                               rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("with_grad", [False, True])
@pytest.mark.parametrize("shape", [(16, 4), (9000, 4)], ids=["few-rows", "many-rows"])
def test_index_cross_entropy_out_of_bounds_status(ctx, shape, with_grad):
    R, C = shape
    pb = ProgramBuilder()
    sx, sy = pb.input(R * C), pb.input(R, "i64")
    sl = pb.output(1)
    sg = pb.output(R * C) if with_grad else None
    pb.index_ce(sx, sy, sl, R, C, grad=sg)
    outs = [sl] + ([sg] if with_grad else [])
    y = np.zeros(R, np.int64)
    y[9] = 4
    with pytest.raises(HipIndexError):
        run_program(ctx, pb, [np.zeros(R * C, np.float32), y], outs)
    y[9] = -1
    with pytest.raises(HipIndexError):
        run_program(ctx, pb, [np.zeros(R * C, np.float32), y], outs)


@pytest.mark.parametrize("mode", ["graph", "direct", "profiled", "async"])
def test_status_word_does_not_leak_between_runs(ctx, mode):
    """A run that flags the status word (an out-of-bounds target) fails; the next run of the same
    program with valid targets succeeds with the right loss, and failing and succeeding runs
    alternate (each run's status is published and cleared by its own last launch)."""
    R, C = 64, 5
    pb = ProgramBuilder()
    sx, sy, sl = pb.input(R * C), pb.input(R, "i64"), pb.output(1)
    pb.index_ce(sx, sy, sl, R, C)
    prog = HipProgram(ctx, pb.image())
    prog.set_graph_mode(mode == "graph")
    prog.set_profiling(mode == "profiled")
    rng = np.random.default_rng(5)
    x = rng.standard_normal((R, C)).astype(np.float32)
    good = rng.integers(0, C, R).astype(np.int64)
    bad = good.copy()
    bad[R - 1] = C
    bx, bgood, bbad, bl = ctx.upload(x), ctx.upload(good), ctx.upload(bad), ctx.buffer(4)
    want = oracle.index_ce_mean(x, good)

    def run(labels):
        if mode == "async":
            prog.run_async([bx, labels], [bl])
            prog.wait()
        else:
            prog.run([bx, labels], [bl])

    for _ in range(3):
        with pytest.raises(HipIndexError):
            run(bbad)
        run(bgood)
        got = bl.download(np.float32, 1)[0]
        assert abs(got - want) <= 1e-5 * abs(want)
    run(bgood)
    prog.close()


# ---- optimizers ----
def _opt_program(ctx, kind, n, **kw):
    pb = ProgramBuilder()
    p = pb.input(n, inout=True)
    g = pb.input(n)
    m = pb.input(n, inout=True)
    v = pb.input(n, inout=True)
    counter = pb.input(1, "i64", inout=True)
    ent = [(p, g, m, v if kind != "sgd" else None, n)]
    pb.optimizer(counter, ent, kind=kind, phase=0, **kw)
    pb.optimizer(counter, ent, kind=kind, phase=1, **kw)
    pb.step_commit(counter)
    return HipProgram(ctx, pb.image())


@pytest.mark.parametrize("cfg", [dict(lr=0.1), dict(lr=0.05, momentum=0.9, has_momentum_slot=True),
                                 dict(lr=0.05, momentum=0.9, nesterov=True, weight_decay=0.01, has_momentum_slot=True),
                                 dict(lr=0.02, momentum=0.5, dampening=0.25, weight_decay=0.1, has_momentum_slot=True)])
def test_sgd_kernel_bit_exact_over_steps(ctx, cfg):
    n = 100_003
    rng = np.random.default_rng(10)
    p0 = rng.standard_normal(n).astype(np.float32)
    prog = _opt_program(ctx, "sgd", n, **cfg)
    bp, bm, bv = ctx.upload(p0), ctx.upload(np.zeros(n, np.float32)), ctx.upload(np.zeros(n, np.float32))
    bc = ctx.upload(np.zeros(1, np.int64))
    p, m = p0.copy(), np.zeros(n, np.float32)
    for step in range(3):
        g = rng.standard_normal(n).astype(np.float32)
        prog.run([bp, ctx.upload(g), bm, bv, bc], [])
        p, m = oracle.sgd_stage(p, g, m, lr=cfg["lr"], momentum=cfg.get("momentum", 0.0),
                                dampening=cfg.get("dampening", 0.0),
                                weight_decay=cfg.get("weight_decay", 0.0),
                                nesterov=cfg.get("nesterov", False), completed_steps=step)
        assert np.array_equal(bp.download(), p)
        if cfg.get("momentum"):
            assert np.array_equal(bm.download(), m)
    assert bc.download(np.int64)[0] == 3


@pytest.mark.parametrize("kind", ["adam", "adamw"])
def test_adam_kernel_over_steps(ctx, kind):
    n = 50_001
    rng = np.random.default_rng(11)
    p0 = rng.standard_normal(n).astype(np.float32)
    kw = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01)
    prog = _opt_program(ctx, kind, n, **kw)
    bp, bm, bv = ctx.upload(p0), ctx.upload(np.zeros(n, np.float32)), ctx.upload(np.zeros(n, np.float32))
    bc = ctx.upload(np.zeros(1, np.int64))
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for step in range(4):
        g = rng.standard_normal(n).astype(np.float32)
        prog.run([bp, ctx.upload(g), bm, bv, bc], [])
        p, m, v = oracle.adam_stage(p, g, m, v, lr=kw["lr"], beta1=kw["beta1"], beta2=kw["beta2"],
                                    eps=kw["eps"], weight_decay=kw["weight_decay"],
                                    decoupled=kind == "adamw", completed_steps=step)
        np.testing.assert_array_max_ulp(bp.download(), p, maxulp=1)
        np.testing.assert_array_max_ulp(bv.download(), v, maxulp=1)


def test_optimizer_non_finite_leaves_state_untouched(ctx):
    n = 5000
    rng = np.random.default_rng(12)
    p0 = rng.standard_normal(n).astype(np.float32)
    prog = _opt_program(ctx, "sgd", n, lr=0.1, momentum=0.9, has_momentum_slot=True)
    bp, bm, bv = ctx.upload(p0), ctx.upload(np.ones(n, np.float32)), ctx.upload(np.zeros(n, np.float32))
    bc = ctx.upload(np.array([5], np.int64))
    g = rng.standard_normal(n).astype(np.float32)
    g[4321] = np.inf
    with pytest.raises(HipArithmeticError):
        prog.run([bp, ctx.upload(g), bm, bv, bc], [])
    assert np.array_equal(bp.download(), p0)
    assert np.array_equal(bm.download(), np.ones(n, np.float32))
    assert bc.download(np.int64)[0] == 5


# ---- benchmark configurations at full size ----
def test_c2_fused_layer_forward_backward_full_size(ctx):
    """C2: Y = ReLU(X.W + b), X [8192,1024] ~ N(0,1), W [1024,1024] Xavier-uniform, b = 0,
    dY ~ N(0,1); Y, dX, dW, db vs the oracle (normwise relative error <= 1e-5; db exact sums)."""
    B, I, O = 8192, 1024, 1024
    rng = np.random.default_rng(20)
    X = rng.standard_normal((B, I)).astype(np.float32)
    bound = math.sqrt(6.0 / (I + O))
    W = rng.uniform(-bound, bound, (I, O)).astype(np.float32)
    b = np.zeros(O, np.float32)
    dY = rng.standard_normal((B, O)).astype(np.float32)
    pb, outs = lower_dense_layer(B, I, O, "relu", "in_out")
    Y, dX, dW, db = run_program(ctx, pb, [X, W, b, dY], list(outs))
    Y = Y.reshape(B, O)
    Yr = oracle.activation("relu", oracle.matmul(X, W))
    # the backward pass differentiates through the forward values it computed, as the reference
    # does: the oracle's backward starts from the GPU's Y, so an activation within rounding of 0
    # (whose mask may differ between two reduction orders) does not change the comparison
    dZ = oracle.activation_grad("relu", dY, Y)
    dXr = oracle.matmul(dZ, W, trans_b=True)
    dWr = oracle.matmul(X, dZ, trans_a=True)
    dbr = oracle.colsum(dZ)
    for got, want in [(Y, Yr), (dX, dXr), (dW, dWr), (db, dbr)]:
        rel = np.linalg.norm(got.reshape(want.shape) - want) / np.linalg.norm(want)
        assert rel <= 1e-5, rel
    # the ReLU mask (a predicate result) is exact wherever the pre-activation is farther from 0
    # than the GEMM's error bound 2 gamma_K sum|x||w|
    u = 2.0 ** -24
    bound = 2 * (I * u / (1 - I * u)) * (np.abs(X).astype(np.float64) @ np.abs(W).astype(np.float64))
    pre = oracle.matmul(X, W)
    decided = np.abs(pre) > bound
    assert decided.mean() > 0.99
    assert np.array_equal((Y > 0)[decided], (Yr > 0)[decided])


def test_c5_softmax_stress_full_size(ctx):
    """C5: row softmax + LSE + mean over [65536, 4096] logits ~ N(0, 4) with 1% entries at +-30,
    forward and backward (dP ~ N(0,1), dm = 1). Size-independent properties on every row,
    the oracle on a sample of rows."""
    R, C = 65536, 4096
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((R, C), dtype=np.float32) * 2)
    mask = rng.random((R, C), dtype=np.float32) < 0.01
    x[mask] = np.where(rng.random(int(mask.sum())) < 0.5, 30.0, -30.0).astype(np.float32)
    dP = rng.standard_normal((R, C), dtype=np.float32)
    pb = ProgramBuilder()
    sx, sdp = pb.input(R * C), pb.input(R * C)
    sp, sl, sm, sdx = pb.output(R * C), pb.output(R), pb.output(1), pb.output(R * C)
    pb.softmax(sx, sp, R, C, lse=sl)
    pb.reduce_all(sl, sm, R, "mean")
    pb.softmax_bwd(sp, sdp, sdx, R, C, rowscale_const=1.0 / R)
    P, L, mean, dX = run_program(ctx, pb, [x, dP], [sp, sl, sm, sdx])
    P = P.reshape(R, C)
    dX = dX.reshape(R, C)
    assert np.isfinite(P).all() and (P >= 0).all()
    np.testing.assert_allclose(P.sum(1, dtype=np.float64), 1.0, rtol=2e-5)
    assert abs(mean[0] - L.astype(np.float64).mean()) <= 1e-6 * abs(mean[0])
    rows = rng.choice(R, 64, replace=False)
    np.testing.assert_allclose(P[rows], oracle.softmax_rows(x[rows]), rtol=2e-6, atol=1e-30)
    np.testing.assert_allclose(L[rows], oracle.logsumexp_rows(x[rows]), rtol=1e-6)
    ref_dx = oracle.softmax_grad_rows(P[rows], dP[rows]) + np.float32(1.0 / R) * P[rows]
    np.testing.assert_allclose(dX[rows], ref_dx, rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("C", [8, 4096, 5000])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_special_rows(ctx, C, log):
    """Rows whose statistics need Math.max semantics (NaN with +inf, zero maxima of either sign,
    -inf with NaN, a subnormal sum) in the register-resident kernels."""
    rng = np.random.default_rng(C + 3)
    x = (rng.standard_normal((10, C)) * 2).astype(np.float32)
    x[0, 1], x[0, 3] = np.inf, np.nan              # NaN beats +inf: everything NaN
    x[1, :] = -np.abs(x[1, :]); x[1, 2] = 0.0       # +0 maximum
    x[2, :] = -np.abs(x[2, :]) - 1; x[2, 5] = -0.0  # -0 maximum
    x[3, :] = -np.abs(x[3, :]); x[3, 0] = 0.0; x[3, 4] = -0.0
    x[4, 0], x[4, 6] = -np.inf, np.nan              # -inf with NaN
    x[5, :] = -np.inf; x[5, 2] = -100.0             # unshifted row with a subnormal sum
    x[6, :] = np.nan
    x[7, 1] = np.inf                                # +inf class rule
    x[8, :] = -np.inf; x[8, 3] = 80.0; x[8, 7] = 85.0  # unshifted, large finite sum
    got, lse = gpu_softmax(ctx, x, log=log)
    want = oracle.softmax_rows(x, log=log)
    want_lse = oracle.logsumexp_rows(x)
    for g_row, w_row in ((got, want), (lse[:, None], want_lse[:, None])):
        nan_w = np.isnan(w_row)
        assert np.array_equal(np.isnan(g_row), nan_w)
        inf_w = np.isinf(w_row)
        assert np.array_equal(g_row[inf_w], w_row[inf_w])
        fin = ~nan_w & ~inf_w
        np.testing.assert_allclose(g_row[fin], w_row[fin], rtol=2e-6, atol=2e-6 if log else 1e-30)
        zero = fin & (w_row == 0)
        assert np.array_equal(np.signbit(g_row[zero]), np.signbit(w_row[zero]))


# ---- single-op pointwise kernels ----
SINGLE_OPS = ["add", "sub", "mul", "div", "max", "gt", "relu_grad", "tanh_grad", "sigmoid_grad",
              "neg", "relu", "tanh", "sigmoid", "exp", "log", "sqrt"]
UNARY = {"neg", "relu", "tanh", "sigmoid", "exp", "log", "sqrt"}


@pytest.mark.parametrize("n", [3, 4, 10007, 3 * 8 * 256 * 4 + 5])
@pytest.mark.parametrize("op", SINGLE_OPS)
def test_single_op_kernel_matches_interpreter(ctx, op, n):
    """A LOAD [LOAD] OP STORE chain runs on the dedicated single-op kernel; the same chain with
    one extra (unused) CONST instruction runs on the interpreter. Both must agree bit for bit,
    special values included."""
    rng = np.random.default_rng(n)
    special = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-40, 3e38, 1.0, -1.0],
                       np.float32)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    y = (rng.standard_normal(n) * 3).astype(np.float32)
    x[: min(n, 10)] = special[: min(n, 10)]
    y[: min(n, 10)] = special[::-1][: min(n, 10)]
    outs = []
    for extra in (False, True):
        pb = ProgramBuilder()
        sx, sy, so = pb.input(n), pb.input(n), pb.output(n)
        code = [("load", 0, 0, 0, 0, 0.0), ("load", 1, 1, 0, 0, 0.0)]
        if extra:
            code.append(("const", 5, 0, 0, 0, 2.0))
        code += [(op, 2, 0, 0 if op in UNARY else 1, 0, 0.0), ("store", 0, 2, 0, 0, 0.0)]
        pb.pointwise(1, n, [sx, sy], [so], code)
        (o,) = run_program(ctx, pb, [x, y], [so])
        outs.append(o.view(np.uint32))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("C", [4096, 4092, 1000, 2048])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_many_rows_special_rows(ctx, C, log):
    """More rows than the device holds workgroups at once, so each workgroup of the row kernels
    takes several rows (an odd or even count) and prefetches the next one; the special-value
    rows sit at positions that fall on either LDS slot of a workgroup's row sequence."""
    R = 3001
    rng = np.random.default_rng(C * 7 + int(log))
    x = (rng.standard_normal((R, C)) * 2).astype(np.float32)
    x[rng.random(x.shape) < 0.01] = 30.0
    for base in (0, 1025, 2050, 2990):
        x[base + 0, 1], x[base + 0, 3] = np.inf, np.nan
        x[base + 1, :] = -np.abs(x[base + 1, :]); x[base + 1, 2] = 0.0
        x[base + 2, :] = -np.abs(x[base + 2, :]) - 1; x[base + 2, 5] = -0.0
        x[base + 3, 1] = np.inf
        x[base + 4, 0] = -np.inf
        x[base + 5, :] = -np.inf; x[base + 5, 3] = 80.0; x[base + 5, 7] = 85.0
        x[base + 6, :] = np.nan
    got, lse = gpu_softmax(ctx, x, log=log)
    want = oracle.softmax_rows(x, log=log)
    want_lse = oracle.logsumexp_rows(x)
    for g_row, w_row in ((got, want), (lse[:, None], want_lse[:, None])):
        nan_w = np.isnan(w_row)
        assert np.array_equal(np.isnan(g_row), nan_w)
        inf_w = np.isinf(w_row)
        assert np.array_equal(g_row[inf_w], w_row[inf_w])
        fin = ~nan_w & ~inf_w
        np.testing.assert_allclose(g_row[fin], w_row[fin], rtol=2e-6, atol=2e-6 if log else 1e-30)
