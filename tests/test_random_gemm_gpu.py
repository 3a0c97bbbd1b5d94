"""Seeded random GEMMs on the GPU against the oracle: shapes drawn so that every route occurs
(K = 1, small K, narrow M or N, ragged edges, aligned and unaligned extents, large enough for the
direct-to-LDS kernel and its in-workgroup split-K, split-K), all four operand layouts, leading
dimensions padded beyond the extents, and the epilogues (bias + activation, activation gradient
with the column sum of the stored result, accumulation into the existing output). Integer-valued
operands make every sum exact, so the GEMM part is bit-exact whatever the reduction order."""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.native import HipProgram
from synaptik_amd.program import ProgramBuilder
from tests.gpu_helpers import run_program

pytestmark = pytest.mark.gpu

EXTENTS = [1, 2, 3, 4, 5, 10, 16, 17, 31, 64, 65, 100, 128, 255, 256, 300, 513, 1024]


def _strided(rng, rows, cols, ld):
    """A rows x cols integer matrix stored with leading dimension ld (>= cols) and the flat
    storage holding it (padding filled with a sentinel that must never be read)."""
    m = rng.integers(-3, 4, size=(rows, cols)).astype(np.float32)
    flat = np.full(rows * ld, 1e30, np.float32)
    for r in range(rows):
        flat[r * ld:r * ld + cols] = m[r]
    if rows:
        flat = flat[: (rows - 1) * ld + cols]
    return m, flat


@pytest.mark.parametrize("seed", range(96))
def test_random_gemm(ctx, seed):
    rng = np.random.default_rng(7000 + seed)
    M, N, K = (int(rng.choice(EXTENTS)) for _ in range(3))
    if rng.random() < 0.25:
        K = int(rng.integers(512, 2300))  # long contractions: split-K and in-workgroup split
        M, N = min(M, 300), min(N, 300)   # (keeps the oracle's sequential product fast)
    ta, tb = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    pad = lambda n: n + int(rng.choice([0, 0, 1, 4, 7]))
    lda = pad(M if ta else K)
    ldb = pad(K if tb else N)
    ldc = pad(N)
    mode = int(rng.integers(0, 3))  # 0 bias + act, 1 act gradient (+ column sum), 2 accumulate
    act = rng.choice(["relu", "tanh", "sigmoid", None]) if mode != 1 else rng.choice(["relu", "tanh", "sigmoid"])
    print(f"gemm seed={seed} M={M} N={N} K={K} ta={ta} tb={tb} lda={lda} ldb={ldb} ldc={ldc} "
          f"mode={mode} act={act}", flush=True)
    A, a_flat = _strided(rng, K if ta else M, M if ta else K, lda)
    B, b_flat = _strided(rng, N if tb else K, K if tb else N, ldb)
    prod = oracle.matmul(A, B, trans_a=ta, trans_b=tb)  # exact: integer operands
    pb = ProgramBuilder()
    sa, sb = pb.input(a_flat.size), pb.input(b_flat.size)
    c0 = rng.integers(-5, 6, size=(M, N)).astype(np.float32)
    _, c_flat = _strided(np.random.default_rng(seed), M, N, ldc)
    for r in range(M):
        c_flat[r * ldc:r * ldc + N] = c0[r]
    inputs = [a_flat, b_flat]
    if mode == 0:
        bias = (rng.integers(-4, 5, N) * 0.25).astype(np.float32)
        sbias = pb.input(N)
        inputs.append(bias)
        sc = pb.output(c_flat.size)
        pb.gemm(sa, sb, sc, M, N, K, trans_a=ta, trans_b=tb, lda=lda, ldb=ldb, ldc=ldc,
                bias=sbias, act=act)
        (out,) = run_program(ctx, pb, inputs, [sc])
        want = oracle.activation(act, (prod + bias[None, :]).astype(np.float32)) if act else \
            (prod + bias[None, :]).astype(np.float32)
    elif mode == 1:
        y = oracle.activation(act, rng.standard_normal((M, N)).astype(np.float32))
        say = pb.input(M * N)
        inputs.append(y)
        sc, scol = pb.output(c_flat.size), pb.output(N)
        pb.gemm(sa, sb, sc, M, N, K, trans_a=ta, trans_b=tb, lda=lda, ldb=ldb, ldc=ldc,
                aux=say, act=act, act_grad=True, colsum=scol)
        out, col = run_program(ctx, pb, inputs, [sc, scol])
        want = oracle.activation_grad(act, prod, y)
        np.testing.assert_array_max_ulp(col, oracle.colsum(want), maxulp=1)
    else:
        sc = pb.input(c_flat.size, inout=True)
        inputs.append(c_flat)
        pb.gemm(sa, sb, sc, M, N, K, trans_a=ta, trans_b=tb, lda=lda, ldb=ldb, ldc=ldc,
                accumulate=True)
        (out,) = _run_inout(ctx, pb, inputs, sc)
        want = (c0 + prod).astype(np.float32)
    got = np.stack([out[r * ldc:r * ldc + N] for r in range(M)]) if M else np.zeros((0, N))
    assert np.array_equal(got.view(np.uint32), np.asarray(want, np.float32).view(np.uint32))


def _run_inout(ctx, pb, inputs, slot):
    """Runs a program whose result is its last (in-place) input and downloads that input."""
    prog = HipProgram(ctx, pb.image())
    bufs = [ctx.upload(np.ascontiguousarray(a)) for a in inputs]
    prog.run(bufs, [])
    out = bufs[-1].download(np.float32, slot.count)
    prog.close()
    return (out,)
