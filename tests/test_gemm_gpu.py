"""GEMM parity on the GPU against the no-FMA sequential oracle (CpuMatmulReferenceKernel).

Integer-valued operands in [-3, 3] make every partial sum exact in binary32, so the MFMA GEMM
must be bit-identical to the oracle whatever its reduction order; N(0,1) operands are checked
against the oracle within the bound |err| <= gamma_K * sum|a||b| (gamma_K = K u / (1 - K u)).
"""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.program import ProgramBuilder
from tests.gpu_helpers import run_program

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1, 1), (7, 5, 3), (64, 64, 16), (256, 64, 16), (256, 1, 64), (130, 70, 33),
          (1024, 10, 1024), (257, 513, 129), (512, 512, 512), (1024, 1024, 784)]


def _gemm_case(ctx, A, B, M, N, K, ta, tb, bias=None, act=None, aux=None, act_grad=False):
    pb = ProgramBuilder()
    sa = pb.input(A.size)
    sb = pb.input(B.size)
    inputs = [A, B]
    sbias = saux = None
    if bias is not None:
        sbias = pb.input(bias.size)
        inputs.append(bias)
    if aux is not None:
        saux = pb.input(aux.size)
        inputs.append(aux)
    sc = pb.output(M * N)
    pb.gemm(sa, sb, sc, M, N, K, trans_a=ta, trans_b=tb, bias=sbias, act=act, aux=saux,
            act_grad=act_grad)
    (C,) = run_program(ctx, pb, inputs, [sc])
    return C.reshape(M, N)


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_gemm_integer_operands_bit_exact(ctx, shape, ta, tb):
    M, N, K = shape
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    A = rng.integers(-3, 4, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K) if tb else (K, N)).astype(np.float32)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb)
    ref = oracle.matmul(A, B, trans_a=ta, trans_b=tb)
    assert np.array_equal(C, ref), f"max diff {np.abs(C - ref).max()}"


@pytest.mark.parametrize("ta,tb", [(False, True), (False, False), (True, False)])
@pytest.mark.parametrize("shape", [(300, 200, 1000), (1024, 1024, 1024)])
def test_gemm_gaussian_within_bound(ctx, shape, ta, tb):
    M, N, K = shape
    rng = np.random.default_rng(5)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb)
    ref = oracle.matmul(A, B, trans_a=ta, trans_b=tb)
    Ad = np.abs(A.T if ta else A).astype(np.float64)
    Bd = np.abs(B.T if tb else B).astype(np.float64)
    u = 2.0 ** -24
    gamma = K * u / (1 - K * u)
    bound = 2 * gamma * (Ad @ Bd) + 1e-30  # GPU and oracle each within gamma of the exact value
    assert (np.abs(C.astype(np.float64) - ref) <= bound).all()
    rel = np.linalg.norm(C - ref) / np.linalg.norm(ref)
    assert rel < 1e-5


@pytest.mark.parametrize("act", ["relu", "tanh", "sigmoid", None])
def test_gemm_bias_activation_epilogue(ctx, act):
    M, N, K = 200, 96, 64
    rng = np.random.default_rng(11)
    X = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(N, K)).astype(np.float32) * np.float32(0.125)
    b = rng.standard_normal(N).astype(np.float32)
    Y = _gemm_case(ctx, X, W, M, N, K, False, True, bias=b, act=act)
    ref = oracle.linear_forward(X, W, b, act)
    assert np.array_equal(Y, ref)


@pytest.mark.parametrize("act", ["relu", "tanh", "sigmoid"])
def test_gemm_activation_gradient_epilogue(ctx, act):
    M, N, K = 130, 72, 48  # dX[M,N] = dZ[M,K] . W[K,N], then act_grad with y = aux
    rng = np.random.default_rng(12)
    dZ = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    y = oracle.activation(act, rng.standard_normal((M, N)).astype(np.float32))
    y[0, :5] = 0.0
    out = _gemm_case(ctx, dZ, W, M, N, K, False, False, aux=y, act=act, act_grad=True)
    ref = oracle.activation_grad(act, oracle.matmul(dZ, W), y)
    assert np.array_equal(out, ref)


def test_gemm_empty_contraction_is_positive_zero(ctx):
    M, N = 5, 7
    A = np.zeros((M, 0), np.float32)
    B = np.zeros((0, N), np.float32)
    pb = ProgramBuilder()
    sa = pb.input(1)
    sb = pb.input(1)
    sc = pb.output(M * N)
    pb.gemm(sa, sb, sc, M, N, 0)
    (C,) = run_program(ctx, pb, [np.zeros(1, np.float32), np.zeros(1, np.float32)], [sc])
    assert np.array_equal(C.view(np.uint32), np.zeros(M * N, np.uint32))


@pytest.mark.parametrize("act", ["relu", "tanh", None])
@pytest.mark.parametrize("K", [1000, 4096])
def test_split_k_epilogues(ctx, act, K):
    """Shapes with too few tiles for the chip take the split-K path (slices reduced in a fixed
    order): integer operands keep it bit-exact, with the bias/activation applied after the sum."""
    M, N = 200, 96
    rng = np.random.default_rng(K)
    X = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(N, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    Y = _gemm_case(ctx, X, W, M, N, K, False, True, bias=b, act=act)
    assert np.array_equal(Y, oracle.linear_forward(X, W, b, act))


def test_split_k_activation_gradient(ctx):
    M, N, K = 130, 72, 2048
    rng = np.random.default_rng(13)
    dZ = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    y = oracle.activation("sigmoid", rng.standard_normal((M, N)).astype(np.float32))
    out = _gemm_case(ctx, dZ, W, M, N, K, False, False, aux=y, act="sigmoid", act_grad=True)
    assert np.array_equal(out, oracle.activation_grad("sigmoid", oracle.matmul(dZ, W), y))


@pytest.mark.parametrize("shape", [(4096, 512, 256), (1000, 300, 64), (130, 72, 2048), (8192, 1024, 1024)])
def test_fused_bias_gradient_column_sum(ctx, shape):
    """GEMM with the activation-gradient epilogue and the SUM_TO_SHAPE of the stored result fused
    (or, for split-K shapes, summed in a separate pass): column sums within 1 ulp of the exact sum."""
    M, N, K = shape
    rng = np.random.default_rng(M + N + K)
    dZ = rng.standard_normal((M, K)).astype(np.float32)
    W = rng.standard_normal((K, N)).astype(np.float32) * np.float32(0.05)
    y = oracle.activation("relu", rng.standard_normal((M, N)).astype(np.float32))
    pb = ProgramBuilder()
    sa, sb, sy = pb.input(M * K), pb.input(K * N), pb.input(M * N)
    sc, sd = pb.output(M * N), pb.output(N)
    pb.gemm(sa, sb, sc, M, N, K, aux=sy, act="relu", act_grad=True, colsum=sd)
    C, db = run_program(ctx, pb, [dZ, W, y], [sc, sd])
    C = C.reshape(M, N)
    np.testing.assert_array_max_ulp(db, oracle.colsum(C), maxulp=1)
    ref = oracle.activation_grad("relu", oracle.matmul(dZ, W), y)
    assert np.linalg.norm(C - ref) / np.linalg.norm(ref) < 1e-5


# Shapes that take the large-problem kernel (M, N multiples of 128 with >= 256 output tiles,
# K a multiple of 32; direct-to-LDS copies, 16x16x4 MFMA): odd and even numbers of k-tiles.
V2_SHAPES = [(2048, 2048, 96), (2048, 4096, 64), (4096, 2048, 32)]


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("shape", V2_SHAPES)
def test_large_tile_kernel_integer_bit_exact(ctx, shape, ta, tb):
    M, N, K = shape
    rng = np.random.default_rng(M + 3 * N + 7 * K + 2 * ta + tb)
    A = rng.integers(-3, 4, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K) if tb else (K, N)).astype(np.float32)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb)
    ref = oracle.matmul(A, B, trans_a=ta, trans_b=tb)
    assert np.array_equal(C, ref), f"max diff {np.abs(C - ref).max()}"


@pytest.mark.parametrize("ta,tb", [(False, True), (False, False), (True, False)])
def test_large_tile_kernel_gaussian_within_bound(ctx, ta, tb):
    M, N, K = 2048, 2048, 512
    rng = np.random.default_rng(17)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb)
    ref = oracle.matmul(A, B, trans_a=ta, trans_b=tb)
    Ad = np.abs(A.T if ta else A).astype(np.float64)
    Bd = np.abs(B.T if tb else B).astype(np.float64)
    u = 2.0 ** -24
    bound = 2 * (K * u / (1 - K * u)) * (Ad @ Bd) + 1e-30
    assert (np.abs(C.astype(np.float64) - ref) <= bound).all()
    assert np.linalg.norm(C - ref) / np.linalg.norm(ref) < 1e-5


@pytest.mark.parametrize("act", ["relu", "tanh", None])
def test_large_tile_kernel_bias_activation(ctx, act):
    M, N, K = 2048, 2048, 64
    rng = np.random.default_rng(23)
    X = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(N, K)).astype(np.float32) * np.float32(0.125)
    b = rng.standard_normal(N).astype(np.float32)
    Y = _gemm_case(ctx, X, W, M, N, K, False, True, bias=b, act=act)
    assert np.array_equal(Y, oracle.linear_forward(X, W, b, act))


@pytest.mark.parametrize("act", ["relu", "sigmoid"])
def test_large_tile_kernel_activation_gradient_and_column_sum(ctx, act):
    M, N, K = 2048, 2048, 64
    rng = np.random.default_rng(29)
    dZ = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    y = oracle.activation(act, rng.standard_normal((M, N)).astype(np.float32))
    pb = ProgramBuilder()
    sa, sb, sy = pb.input(M * K), pb.input(K * N), pb.input(M * N)
    sc, sd = pb.output(M * N), pb.output(N)
    pb.gemm(sa, sb, sc, M, N, K, aux=sy, act=act, act_grad=True, colsum=sd)
    C, db = run_program(ctx, pb, [dZ, W, y], [sc, sd])
    C = C.reshape(M, N)
    assert np.array_equal(C, oracle.activation_grad(act, oracle.matmul(dZ, W), y))
    np.testing.assert_array_max_ulp(db, oracle.colsum(C), maxulp=1)


def test_large_tile_kernel_accumulate(ctx):
    M, N, K = 2048, 2048, 32
    rng = np.random.default_rng(31)
    A = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K)).astype(np.float32)
    C0 = rng.integers(-8, 9, size=(M, N)).astype(np.float32)
    pb = ProgramBuilder()
    sa, sb, sc = pb.input(M * K), pb.input(N * K), pb.output(M * N)
    pb.copy(pb.input(M * N), sc, M * N)
    pb.gemm(sa, sb, sc, M, N, K, trans_b=True, accumulate=True)
    (C,) = run_program(ctx, pb, [A, B, C0], [sc])
    assert np.array_equal(C.reshape(M, N), C0 + oracle.matmul(A, B, trans_b=True))


@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (False, False)])
def test_large_tile_kernel_split_k(ctx, ta, tb):
    """Few output tiles and a long K: split-K slices on the large-problem kernel, reduced in slice
    order; integer operands keep it bit-exact, bias and ReLU applied after the reduction."""
    M, N, K = 1024, 1024, 4096
    rng = np.random.default_rng(37 + ta + 2 * tb)
    A = rng.integers(-3, 4, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K) if tb else (K, N)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb, bias=b, act="relu")
    Z = oracle.matmul(A, B, trans_a=ta, trans_b=tb)
    assert np.array_equal(C, oracle.activation("relu", Z + b))


def test_large_tile_kernel_strided_operands_and_output(ctx):
    """Leading dimensions wider than the logical extents (a column block of wider storage for A,
    B and C, and of the aux operand): the large-problem kernel reads and writes only the block."""
    M, N, K = 2048, 2048, 64
    lda, ldb, ldc = K + 32, N + 128, N + 64
    rng = np.random.default_rng(41)
    A = rng.integers(-3, 4, size=(M, lda)).astype(np.float32)
    B = rng.integers(-3, 4, size=(K, ldb)).astype(np.float32)
    y = oracle.activation("relu", rng.standard_normal((M, ldc)).astype(np.float32))
    C0 = np.full((M, ldc), 7.0, np.float32)
    pb = ProgramBuilder()
    sa, sb, sy = pb.input(A.size), pb.input(B.size), pb.input(y.size)
    sc = pb.output(C0.size)
    pb.copy(pb.input(C0.size), sc, C0.size)
    pb.gemm(sa, sb, sc, M, N, K, lda=lda, ldb=ldb, ldc=ldc, aux=sy, ldaux=ldc, act="relu",
            act_grad=True)
    (C,) = run_program(ctx, pb, [A, B, y, C0], [sc])
    C = C.reshape(M, ldc)
    Z = oracle.matmul(np.ascontiguousarray(A[:, :K]), np.ascontiguousarray(B[:, :N]))
    assert np.array_equal(C[:, :N], oracle.activation_grad("relu", Z, np.ascontiguousarray(y[:, :N])))
    assert (C[:, N:] == 7.0).all()


# Shapes for the 64x64 direct-to-LDS tiles (no split-K) and the ragged-edge (TAIL) variants:
# whole tiles; ragged K (784 = 24.5 k-tiles); ragged N (784); ragged M, N and K together; a
# ragged split-K problem on 128x128 tiles.
EDGE_SHAPES = [(1024, 1024, 1024), (1024, 1024, 784), (1024, 784, 1024), (1000, 1028, 100),
               (4100, 2052, 36), (200, 1024, 4100)]


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("shape", EDGE_SHAPES, ids=str)
def test_direct_lds_kernel_edges_integer_bit_exact(ctx, shape, ta, tb):
    M, N, K = shape
    if ta and M % 4:
        pytest.skip("M-contiguous A needs M % 4 == 0 for 16-byte loads (other kernel)")
    rng = np.random.default_rng(M + 5 * N + 11 * K + 2 * ta + tb)
    A = rng.integers(-3, 4, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K) if tb else (K, N)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb, bias=b, act="relu")
    Z = oracle.matmul(A, B, trans_a=ta, trans_b=tb)
    assert np.array_equal(C, oracle.activation("relu", Z + b)), f"max diff {np.abs(C - oracle.activation('relu', Z + b)).max()}"


@pytest.mark.parametrize("shape", [(1024, 1024, 1024), (1000, 1028, 100)], ids=str)
def test_direct_lds_kernel_edges_gradient_column_sum(ctx, shape):
    M, N, K = shape
    rng = np.random.default_rng(43)
    dZ = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    y = oracle.activation("tanh", rng.standard_normal((M, N)).astype(np.float32))
    pb = ProgramBuilder()
    sa, sb, sy = pb.input(M * K), pb.input(K * N), pb.input(M * N)
    sc, sd = pb.output(M * N), pb.output(N)
    pb.gemm(sa, sb, sc, M, N, K, aux=sy, act="tanh", act_grad=True, colsum=sd)
    C, db = run_program(ctx, pb, [dZ, W, y], [sc, sd])
    C = C.reshape(M, N)
    assert np.array_equal(C, oracle.activation_grad("tanh", oracle.matmul(dZ, W), y))
    np.testing.assert_array_max_ulp(db, oracle.colsum(C), maxulp=1)


# Skinny problems (one of M, N, K <= 16): the small-K, row-dot and column-outer kernels, with
# aligned and unaligned extents, every operand layout, long and short contractions.
SKINNY_SHAPES = [(1, 4096, 4096), (16, 1000, 777), (1000, 16, 513), (3, 5, 100), (17, 16, 2),
                 (4099, 1027, 2), (1024, 1024, 10), (10, 1024, 1024), (5000, 3, 33),
                 (2, 2, 70000), (1, 1, 4096), (16, 16, 17), (33, 1028, 16), (1025, 1, 300)]


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("shape", SKINNY_SHAPES, ids=str)
def test_skinny_integer_operands_bit_exact(ctx, shape, ta, tb):
    M, N, K = shape
    rng = np.random.default_rng(M * 7 + N * 13 + K)
    A = rng.integers(-3, 4, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K) if tb else (K, N)).astype(np.float32)
    print(f"skinny M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb)
    assert np.array_equal(C, oracle.matmul(A, B, trans_a=ta, trans_b=tb))


@pytest.mark.parametrize("ta,tb", [(False, True), (False, False), (True, False), (True, True)])
@pytest.mark.parametrize("shape", [(1024, 10, 1024), (10, 1024, 1024), (1024, 1024, 10),
                                   (1, 4096, 4096), (7, 3, 50000)], ids=str)
def test_skinny_gaussian_within_bound(ctx, shape, ta, tb):
    M, N, K = shape
    rng = np.random.default_rng(17)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb)
    ref = oracle.matmul(A, B, trans_a=ta, trans_b=tb)
    Ad = np.abs(A.T if ta else A).astype(np.float64)
    Bd = np.abs(B.T if tb else B).astype(np.float64)
    u = 2.0 ** -24
    gamma = K * u / (1 - K * u)
    assert (np.abs(C.astype(np.float64) - ref) <= 2 * gamma * (Ad @ Bd) + 1e-30).all()


@pytest.mark.parametrize("act", ["relu", "tanh", "sigmoid", None])
@pytest.mark.parametrize("shape", [(1024, 10, 1024), (1, 4096, 512), (300, 16, 12), (5, 37, 3),
                                   (256, 64, 16), (4097, 128, 9)], ids=str)
def test_skinny_bias_activation_epilogue(ctx, act, shape):
    M, N, K = shape
    rng = np.random.default_rng(23)
    X = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(N, K)).astype(np.float32) * np.float32(0.125)
    b = rng.standard_normal(N).astype(np.float32)
    Y = _gemm_case(ctx, X, W, M, N, K, False, True, bias=b, act=act)
    assert np.array_equal(Y, oracle.linear_forward(X, W, b, act))


@pytest.mark.parametrize("shape", [(1024, 1024, 10), (1000, 1026, 7), (10, 300, 2048), (300, 10, 2048),
                                   (256, 64, 16), (3001, 100, 5), (129, 128, 3)], ids=str)
def test_skinny_activation_gradient_and_column_sum(ctx, shape):
    M, N, K = shape
    rng = np.random.default_rng(29)
    dZ = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    y = oracle.activation("relu", rng.standard_normal((M, N)).astype(np.float32))
    pb = ProgramBuilder()
    sa, sb, sy = pb.input(M * K), pb.input(K * N), pb.input(M * N)
    sc, sd = pb.output(M * N), pb.output(N)
    pb.gemm(sa, sb, sc, M, N, K, aux=sy, act="relu", act_grad=True, colsum=sd)
    C, db = run_program(ctx, pb, [dZ, W, y], [sc, sd])
    ref = oracle.activation_grad("relu", oracle.matmul(dZ, W), y)
    assert np.array_equal(C.reshape(M, N), ref)
    np.testing.assert_array_max_ulp(db, oracle.colsum(ref), maxulp=1)



# In-workgroup split-K (64x64 tiles, fewer than 512 of them, K >= 512): two groups of four waves
# on the two halves of the k-tiles, an odd count zero-filling group 1's last tile.
KS2_SHAPES = [(1024, 1024, 512), (1024, 1024, 544), (960, 1000, 1000), (512, 512, 2048),
              (1000, 1028, 777), (640, 1024, 4096), (1024, 1024, 1024), (1024, 1024, 1056),
              (960, 1000, 2000), (1000, 1028, 1540)]


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("shape", KS2_SHAPES, ids=str)
def test_split_in_group_integer_bit_exact(ctx, shape, ta, tb):
    M, N, K = shape
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    A = rng.integers(-3, 4, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K) if tb else (K, N)).astype(np.float32)
    print(f"ks2 M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb)
    assert np.array_equal(C, oracle.matmul(A, B, trans_a=ta, trans_b=tb))


@pytest.mark.parametrize("shape", [(1024, 1024, 1024), (1000, 1028, 777), (1000, 1028, 1540)],
                         ids=str)
def test_split_in_group_gradient_column_sum(ctx, shape):
    M, N, K = shape
    rng = np.random.default_rng(41)
    dZ = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    y = oracle.activation("relu", rng.standard_normal((M, N)).astype(np.float32))
    pb = ProgramBuilder()
    sa, sb, sy = pb.input(M * K), pb.input(K * N), pb.input(M * N)
    sc, sd = pb.output(M * N), pb.output(N)
    pb.gemm(sa, sb, sc, M, N, K, aux=sy, act="relu", act_grad=True, colsum=sd)
    C, db = run_program(ctx, pb, [dZ, W, y], [sc, sd])
    ref = oracle.activation_grad("relu", oracle.matmul(dZ, W), y)
    assert np.array_equal(C.reshape(M, N), ref)
    np.testing.assert_array_max_ulp(db, oracle.colsum(ref), maxulp=1)


def test_split_in_group_gaussian_within_bound(ctx):
    M, N, K = 1024, 784, 1024
    rng = np.random.default_rng(43)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((N, K)).astype(np.float32)
    C = _gemm_case(ctx, A, B, M, N, K, False, True)
    ref = oracle.matmul(A, B, trans_b=True)
    u = 2.0 ** -24
    gamma = K * u / (1 - K * u)
    bound = 2 * gamma * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64).T) + 1e-30
    assert (np.abs(C.astype(np.float64) - ref) <= bound).all()


# In-workgroup split-K on the split-K slices of 128x128 tiles (fewer than 512 tile slices, slices
# of at least 512 of K): each slice's two K groups are summed in LDS (group 0 + group 1) before
# the slice's partial is stored; ragged last slices zero-fill group 1's missing k-tiles.
KS2_SLICE_SHAPES = [(1024, 1024, 8192), (512, 1024, 8192), (1000, 1028, 5000), (640, 1024, 4096),
                    (1024, 1000, 3000)]


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("shape", KS2_SLICE_SHAPES, ids=str)
def test_split_slices_in_group_integer_bit_exact(ctx, shape, ta, tb):
    M, N, K = shape
    rng = np.random.default_rng(M + 5 * N + 11 * K + ta + 2 * tb)
    A = rng.integers(-3, 4, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K) if tb else (K, N)).astype(np.float32)
    print(f"ks2 slices M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    C = _gemm_case(ctx, A, B, M, N, K, ta, tb)
    assert np.array_equal(C, oracle.matmul(A, B, trans_a=ta, trans_b=tb))


def test_split_slices_in_group_gaussian_bias_relu(ctx):
    M, N, K = 1000, 1028, 5000
    rng = np.random.default_rng(47)
    A = rng.standard_normal((K, M)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    print(f"ks2 slices gaussian M={M} N={N} K={K}", flush=True)
    C = _gemm_case(ctx, A, B, M, N, K, True, False, bias=b, act="relu")
    Z = oracle.matmul(A, B, trans_a=True).astype(np.float64)
    u = 2.0 ** -24
    gamma = K * u / (1 - K * u)
    bound = 2 * gamma * (np.abs(A).astype(np.float64).T @ np.abs(B).astype(np.float64)) + 1e-30
    pre = Z + b
    # where the pre-activation is decided beyond the bound, the ReLU output follows it exactly
    decided = np.abs(pre) > bound + 1e-6 * np.abs(pre)
    want = np.maximum(pre, 0.0)
    assert (np.abs(C.astype(np.float64) - want)[decided] <= (bound + 1e-6 * np.abs(pre))[decided]).all()


@pytest.mark.parametrize("shape", [(1024, 1024, 8192), (1000, 1028, 5000)], ids=str)
def test_split_slices_in_group_gradient_column_sum(ctx, shape):
    """Activation-gradient epilogue and bias-gradient column sum on split-K slices run by eight-wave
    workgroups: applied by the slice reduction after the slices are added in order."""
    M, N, K = shape
    rng = np.random.default_rng(53)
    dZ = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    W = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    y = oracle.activation("relu", rng.standard_normal((M, N)).astype(np.float32))
    pb = ProgramBuilder()
    sa, sb, sy = pb.input(M * K), pb.input(K * N), pb.input(M * N)
    sc, sd = pb.output(M * N), pb.output(N)
    pb.gemm(sa, sb, sc, M, N, K, aux=sy, act="relu", act_grad=True, colsum=sd)
    print(f"ks2 slices gradient M={M} N={N} K={K}", flush=True)
    C, db = run_program(ctx, pb, [dZ, W, y], [sc, sd])
    ref = oracle.activation_grad("relu", oracle.matmul(dZ, W), y)
    assert np.array_equal(C.reshape(M, N), ref)
    np.testing.assert_array_max_ulp(db, oracle.colsum(ref), maxulp=1)
