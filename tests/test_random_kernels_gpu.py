"""Seeded random shapes for the reduction, softmax and loss kernels on the GPU against the oracle:
extents from 1 to several thousand (multiples of 4 and not, below and above the register-resident
row limit, narrow and wide column sums, padded row strides), special values mixed in, both
reductions of MSE, CE with and without an ignore index over int32 and int64 targets. Bounds as in
the fixed-shape tests: sums and means within 1 ulp of the exactly rounded result, softmax within
2e-6 relative, losses within 1e-5 relative, gradients bit-exact where the arithmetic is."""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.program import ProgramBuilder
from tests.gpu_helpers import run_program

pytestmark = pytest.mark.gpu

DIMS = [1, 2, 3, 4, 7, 10, 63, 64, 65, 255, 256, 1000, 1023, 1024, 2049, 4096, 4097, 5003]


@pytest.mark.parametrize("seed", range(32))
def test_random_colsum(ctx, seed):
    rng = np.random.default_rng(100 + seed)
    R = int(rng.choice(DIMS + [20000, 40000]))
    N = int(rng.choice(DIMS[:14]))
    ldx = N + int(rng.choice([0, 0, 1, 4, 13]))
    mean, acc = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    print(f"colsum seed={seed} R={R} N={N} ldx={ldx} mean={mean} acc={acc}", flush=True)
    x = rng.standard_normal((R, ldx)).astype(np.float32)
    x[:, N:] = np.nan  # padding: must never be read
    old = rng.standard_normal(N).astype(np.float32)
    pb = ProgramBuilder()
    sx = pb.input(R * ldx)
    so = pb.input(N, inout=True) if acc else pb.output(N)
    pb.colsum(sx, so, R, N, ldx=ldx, mean=mean, accumulate=acc)
    if acc:
        from synaptik_amd.native import HipProgram
        prog = HipProgram(ctx, pb.image())
        bx, bo = ctx.upload(x.ravel()), ctx.upload(old)
        prog.run([bx, bo], [])
        got = bo.download(np.float32, N)
        prog.close()
    else:
        (got,) = run_program(ctx, pb, [x.ravel()], [so])
    cols = x[:, :N]
    part = np.array([oracle.exact_mean(cols[:, c]) if mean else oracle.exact_sum(cols[:, c])
                     for c in range(N)], np.float32)
    if acc:
        # the GPU adds the new column sum to the old value once (binary32), as the reference's
        # accumulation does; the sum itself may differ from the exact one by 1 ulp
        np.testing.assert_allclose(got, old + part, rtol=2e-6, atol=2e-6 * np.abs(part).max())
    else:
        np.testing.assert_array_max_ulp(got, part, maxulp=1)


@pytest.mark.parametrize("seed", range(24))
def test_random_row_reductions_and_softmax(ctx, seed):
    rng = np.random.default_rng(200 + seed)
    R, C = int(rng.choice([1, 3, 64, 513])), int(rng.choice(DIMS))
    x = (rng.standard_normal((R, C)) * 3).astype(np.float32)
    x[rng.random(x.shape) < 0.005] = 30.0
    if R > 2 and C > 1:
        x[1, 0] = -np.inf
    print(f"rows seed={seed} R={R} C={C}", flush=True)
    pb = ProgramBuilder()
    sx = pb.input(R * C)
    outs = {k: pb.output(R) for k in ("sum", "mean", "max", "lse")}
    for k, s in outs.items():
        pb.row_reduce(sx, s, R, C, k)
    sy, sl, syl = pb.output(R * C), pb.output(R), pb.output(R * C)
    pb.softmax(sx, sy, R, C, lse=sl)
    pb.softmax(sx, syl, R, C, log=True)
    got = dict(zip(list(outs) + ["softmax", "lse2", "log"],
                   run_program(ctx, pb, [x], list(outs.values()) + [sy, sl, syl])))
    np.testing.assert_array_max_ulp(got["sum"], np.array([oracle.exact_sum(r) for r in x], np.float32), maxulp=1)
    np.testing.assert_array_max_ulp(got["mean"], np.array([oracle.exact_mean(r) for r in x], np.float32), maxulp=1)
    assert np.array_equal(got["max"], x.max(axis=1))
    lse = oracle.logsumexp_rows(x)
    np.testing.assert_allclose(got["lse"], lse, rtol=1e-6)
    np.testing.assert_allclose(got["lse2"], lse, rtol=1e-6)
    np.testing.assert_allclose(got["softmax"].reshape(R, C), oracle.softmax_rows(x), rtol=2e-6, atol=1e-30)
    np.testing.assert_allclose(got["log"].reshape(R, C), oracle.softmax_rows(x, log=True), rtol=1e-6, atol=2e-6)


@pytest.mark.parametrize("seed", range(24))
def test_random_losses(ctx, seed):
    rng = np.random.default_rng(300 + seed)
    # MSE over n elements, both reductions
    n = int(rng.choice([1, 3, 1000, 4097, 65536, 1_000_003]))
    red = "sum" if rng.random() < 0.3 else "mean"
    p = rng.standard_normal(n).astype(np.float32)
    t = rng.standard_normal(n).astype(np.float32)
    pb = ProgramBuilder()
    sp, st = pb.input(n), pb.input(n)
    sl, sg = pb.output(1), pb.output(n)
    pb.mse(sp, st, sl, n, grad=sg, reduction=red)
    loss, grad = run_program(ctx, pb, [p, t], [sl, sg])
    assert np.array_equal(grad, oracle.mse_grad(p, t, reduction=red))
    exact = np.sum((p.astype(np.float64) - t) ** 2) / (n if red == "mean" else 1)
    assert abs(loss[0] - exact) <= 1e-6 * abs(exact) + 1e-30
    # index CE
    R, C = int(rng.choice([1, 5, 1024, 4100, 9000])), int(rng.choice([2, 3, 10, 100, 300]))
    ignore = -100 if rng.random() < 0.5 else None
    dt = "i64" if rng.random() < 0.5 else "i32"
    print(f"losses seed={seed} n={n} {red} R={R} C={C} ignore={ignore} {dt}", flush=True)
    logits = (rng.standard_normal((R, C)) * 3).astype(np.float32)
    y = rng.integers(0, C, R)
    if ignore is not None:
        y[rng.random(R) < 0.2] = ignore
        y[0] = 0  # at least one counted sample
    pb = ProgramBuilder()
    sx, sy = pb.input(R * C), pb.input(R, dt)
    sl, sg = pb.output(1), pb.output(R * C)
    pb.index_ce(sx, sy, sl, R, C, grad=sg, ignore_index=ignore)
    loss, grad = run_program(ctx, pb, [logits, y.astype(np.int64 if dt == "i64" else np.int32)], [sl, sg])
    want = oracle.index_ce_mean(logits, y, ignore_index=ignore)
    assert abs(loss[0] - want) <= 1e-5 * abs(want)
    np.testing.assert_allclose(grad.reshape(R, C), oracle.index_ce_grad(logits, y, ignore_index=ignore),
                               rtol=1e-5, atol=1e-9)
