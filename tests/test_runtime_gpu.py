"""Runtime boundary behaviour on the GPU: validation at program create, binding checks at run,
and empty / degenerate shapes (the reference's Metal bridge rejects the same classes of misuse,
synaptik_metal_foundation.m:10012-10020)."""
import math

import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.native import HipBackendError, HipInvalidArgument, HipProgram
from synaptik_amd.program import ProgramBuilder
from tests.gpu_helpers import run_program

pytestmark = pytest.mark.gpu


def test_create_rejects_operands_larger_than_their_slots(ctx):
    pb = ProgramBuilder()
    a, b, c = pb.input(10), pb.input(10), pb.output(9)
    pb.gemm(a, b, c, 4, 3, 3)  # A needs 12 floats, C 12
    with pytest.raises(HipInvalidArgument):
        HipProgram(ctx, pb.image())


def test_create_rejects_writes_to_read_only_inputs_and_bad_images(ctx):
    pb = ProgramBuilder()
    a = pb.input(16)
    b = pb.input(16)
    pb.copy(a, b, 16)
    with pytest.raises(HipBackendError):
        HipProgram(ctx, pb.image())
    with pytest.raises(HipBackendError):
        HipProgram(ctx, b"SHKP" + b"\0" * 8)
    img = bytearray(ProgramBuilder().image())
    img[0] ^= 1
    with pytest.raises(HipBackendError):
        HipProgram(ctx, bytes(img))


def test_run_checks_binding_counts_sizes_and_aliasing(ctx):
    pb = ProgramBuilder()
    x = pb.input(64)
    y = pb.output(64)
    pb.copy(x, y, 64)
    prog = HipProgram(ctx, pb.image())
    bx, by = ctx.upload(np.arange(64, dtype=np.float32)), ctx.buffer(256)
    prog.run([bx], [by])
    assert np.array_equal(by.download(), np.arange(64, dtype=np.float32))
    with pytest.raises(HipInvalidArgument):
        prog.run([bx, bx], [by])
    with pytest.raises(HipInvalidArgument):
        prog.run([ctx.buffer(16)], [by])
    with pytest.raises(HipInvalidArgument):
        prog.run([bx], [bx])  # output aliases an input
    prog.close()


def test_degenerate_shapes(ctx):
    # M = 0 / N = 0 GEMMs, a single-column softmax, an empty sum and mean, C = 1 LSE
    pb = ProgramBuilder()
    a, b = pb.input(4), pb.input(4)
    c0 = pb.output(1)
    pb.gemm(a, b, c0, 0, 1, 4)
    pb.gemm(a, b, c0, 1, 0, 4)
    x = pb.input(5)
    sm, ls = pb.output(5), pb.output(5)
    pb.softmax(x, sm, 5, 1, lse=ls)
    e = pb.input(1)
    s_sum, s_mean, s_max = pb.output(1), pb.output(1), pb.output(1)
    pb.reduce_all(e, s_sum, 0, "sum")
    pb.reduce_all(e, s_mean, 0, "mean")
    pb.reduce_all(e, s_max, 0, "max")
    xs = np.array([3.0, -2.0, np.inf, -np.inf, 0.5], np.float32)
    outs = run_program(ctx, pb, [np.ones(4, np.float32), np.ones(4, np.float32), xs,
                                 np.zeros(1, np.float32)], [c0, sm, ls, s_sum, s_mean, s_max])
    _, p, l, ssum, smean, smax = outs
    want = oracle.softmax_rows(xs.reshape(5, 1)).ravel()
    for g, w in zip(p, want):
        assert (math.isnan(g) and math.isnan(w)) or g == w
    assert ssum[0] == 0.0 and math.isnan(smean[0]) and smax[0] == -np.inf
    np.testing.assert_array_equal(l[[0, 1, 4]], xs[[0, 1, 4]])


def test_cross_entropy_with_every_sample_ignored(ctx):
    R, C = 8, 3
    pb = ProgramBuilder()
    sx, sy = pb.input(R * C), pb.input(R, "i64")
    sl, sg = pb.output(1), pb.output(R * C)
    pb.index_ce(sx, sy, sl, R, C, grad=sg, ignore_index=-1)
    loss, grad = run_program(ctx, pb, [np.ones(R * C, np.float32), np.full(R, -1, np.int64)], [sl, sg])
    assert math.isnan(loss[0])  # 0 / 0, as the reference's sum / count
    assert np.array_equal(grad, np.zeros(R * C, np.float32))


def test_program_is_reusable_and_arena_persists_between_runs(ctx):
    pb = ProgramBuilder()
    x = pb.input(1000)
    t = pb.internal(1000)
    y = pb.output(1)
    pb.copy(x, t, 1000)
    pb.reduce_all(t, y, 1000, "sum")
    prog = HipProgram(ctx, pb.image())
    assert prog.arena_bytes() >= 4000 and prog.step_count() == 2
    for k in range(1, 4):
        bx, by = ctx.upload(np.full(1000, k, np.float32)), ctx.buffer(4)
        prog.run([bx], [by])
        assert by.download()[0] == 1000.0 * k
    prog.set_profiling(True)
    prog.run([bx], [by])
    times, runs = prog.step_times()
    assert runs == 1 and len(times) == 2 and all(t > 0 for t in times)
    prog.close()


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 1_000_003, 1 << 24])
def test_copy_is_bit_exact_for_ragged_lengths(ctx, n):
    # the vector body copies whole float4s, the scalar tail the last n % 4 elements; NaN
    # payloads and signed zeros must come through unchanged (the copy moves bits, not values)
    rng = np.random.default_rng(n)
    bits = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    bits[: min(n, 4)] = [0x7FC00001, 0x80000000, 0xFF800000, 0x00000001][: min(n, 4)]
    src = bits.view(np.float32)
    pb = ProgramBuilder()
    x, y = pb.input(n), pb.output(n + 4)
    pb.fill(y, n + 4, 7.0)
    pb.copy(x, y, n)
    prog = HipProgram(ctx, pb.image())
    bx, by = ctx.upload(src), ctx.buffer((n + 4) * 4)
    prog.run([bx], [by])
    got = by.download().view(np.uint32)
    assert np.array_equal(got[:n], bits)
    assert np.all(by.download()[n:] == 7.0)  # nothing written past the copied range
    prog.close()
