"""A forward GEMM with its cotangent (mode 2): C = act(A.B + b), dZ = act_grad(dY, C) and the column
sums of dZ from one step, on every route -- the direct-to-LDS tile kernel (64- and 128-wide tiles),
the register-staged tile kernel, the skinny kernels, split-K and the K = 1 outer product (the last
three form dZ in a separate pass). C must equal the plain forward GEMM bit for bit, dZ the
activation gradient of the stored C (exactly for ReLU: a selection), and the column sums the
binary64 sum of dZ rounded once."""
import numpy as np
import pytest

from synaptik_amd.program import ProgramBuilder
from tests.gpu_helpers import run_program

pytestmark = pytest.mark.gpu

SHAPES = [
    (1024, 512, 256, False),   # direct-to-LDS, 64-wide tiles
    (2048, 1024, 512, True),   # direct-to-LDS, 128-wide tiles, B transposed
    (100, 36, 50, False),      # register-staged tile kernel (too few tiles for the direct one)
    (96, 37, 40, True),        # N off 4: register-staged, scalar epilogue
    (300, 10, 600, False),     # skinny (narrow N)
    (64, 64, 8192, False),     # split along K
    (200, 48, 1, False),       # K = 1
]


def _act_grad(act, dy, y):
    if act == "relu":
        return np.where(y > 0, dy, np.float32(0))
    if act == "tanh":
        return dy * (np.float32(1) - y * y)
    return (dy * y) * (np.float32(1) - y)


@pytest.mark.parametrize("M,N,K,tb", SHAPES)
@pytest.mark.parametrize("act", ["relu", "tanh", "sigmoid"])
def test_forward_gemm_with_cotangent_on_every_route(ctx, M, N, K, tb, act):
    print(f"[gemm mode 2] M={M} N={N} K={K} transB={tb} act={act}", flush=True)
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    A = rng.standard_normal((M, K), dtype=np.float32)
    B = (rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)
    dY = rng.standard_normal((M, N), dtype=np.float32)

    pb = ProgramBuilder()
    sa, sb, sbias, sdy = pb.input(M * K), pb.input(B.size), pb.input(N), pb.input(M * N)
    sy, sdz, sdb = pb.output(M * N), pb.output(M * N), pb.output(N)
    pb.gemm(sa, sb, sy, M, N, K, trans_b=tb, bias=sbias, act=act, dy=sdy, dz=sdz, colsum=sdb)
    y, dz, db = run_program(ctx, pb, [A, B, b, dY], [sy, sdz, sdb])

    pb = ProgramBuilder()
    sa, sb, sbias = pb.input(M * K), pb.input(B.size), pb.input(N)
    sy0 = pb.output(M * N)
    pb.gemm(sa, sb, sy0, M, N, K, trans_b=tb, bias=sbias, act=act)
    (y0,) = run_program(ctx, pb, [A, B, b], [sy0])

    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32))
    y = y.reshape(M, N)
    dz = dz.reshape(M, N)
    want = _act_grad(act, dY, y)
    if act == "relu":
        assert np.array_equal(dz.view(np.uint32), want.view(np.uint32))
    else:  # the device may contract 1 - y*y (or g*y then * (1 - y)) into one rounding
        np.testing.assert_allclose(dz, want, rtol=4e-7, atol=1e-30)
    np.testing.assert_allclose(db, dz.astype(np.float64).sum(0).astype(np.float32), rtol=1e-6,
                               atol=1e-6)


def test_cotangent_mode_rejects_aliasing_and_missing_slots(ctx):
    from synaptik_amd.native import HipBackendError, HipProgram
    pb = ProgramBuilder()
    a, b, dy = pb.input(16), pb.input(16), pb.input(16)
    y = pb.output(16)
    pb.gemm(a, b, y, 4, 4, 4, act="relu", dy=dy, dz=y)  # dZ aliases C
    with pytest.raises(HipBackendError):
        HipProgram(ctx, pb.image())
    pb = ProgramBuilder()
    a, b = pb.input(16), pb.input(16)
    y, dz = pb.output(16), pb.output(16)
    pb.gemm(a, b, y, 4, 4, 4, act="relu", dy=y, dz=dz)  # dY aliases C
    with pytest.raises(HipBackendError):
        HipProgram(ctx, pb.image())
