"""Staged uploads on the copy stream and asynchronous runs (shk_hip_buffer_upload_staged,
shk_hip_program_run_async / _wait) and the pipelined training loop built on them
(HipTrainingSession.run_pipelined). The bar is the synchronous path itself: bytes land exactly,
every cross-stream order holds (a run sees a staged upload; a staged upload does not overwrite a
buffer a pending run still reads), and a pipelined training loop is bit-identical to one `run`
per batch, failures included."""
import numpy as np
import pytest

from synaptik_amd.native import HipArithmeticError, HipIndexError, HipProgram
from synaptik_amd.program import ProgramBuilder
from synaptik_amd.training import Adam, HipTrainingSession, MlpSpec, Sgd, init_parameters

pytestmark = pytest.mark.gpu

CHUNK = 8 << 20  # the staging ring's chunk size


@pytest.mark.parametrize("nbytes,offset", [(1, 0), (4096, 12), (CHUNK, 0), (CHUNK + 3, 5),
                                           (5 * CHUNK + 17, 0)])
def test_staged_upload_lands_exactly(ctx, nbytes, offset):
    rng = np.random.default_rng(nbytes)
    data = rng.integers(0, 256, nbytes, dtype=np.uint8)
    buf = ctx.buffer(nbytes + offset + 7)
    buf.upload(np.zeros(nbytes + offset + 7, np.uint8))
    buf.upload_staged(data, offset)
    got = buf.download(np.uint8)
    assert np.array_equal(got[offset:offset + nbytes], data)
    assert not got[:offset].any() and not got[offset + nbytes:].any()
    buf.close()


def _neg_program(n):
    pb = ProgramBuilder()
    sx, so = pb.input(n), pb.output(n)
    pb.pointwise(1, n, [sx], [so], [("load", 0, 0, 0, 0, 0.0), ("neg", 1, 0, 0, 0, 0.0),
                                     ("store", 0, 1, 0, 0, 0.0)])
    return pb


def test_run_sees_staged_upload_and_upload_waits_for_pending_run(ctx):
    n = 12 << 20  # 48 MiB: several chunks, long enough for the run to be in flight
    rng = np.random.default_rng(1)
    old = rng.standard_normal(n).astype(np.float32)
    new = rng.standard_normal(n).astype(np.float32)
    prog = HipProgram(ctx, _neg_program(n).image())
    x, out = ctx.buffer(4 * n), ctx.buffer(4 * n)
    x.upload_staged(old)
    prog.run_async([x], [out])       # must read `old` (waits for the staged copy)
    x.upload_staged(new)             # must not land before that run has read x
    prog.wait()
    assert np.array_equal(out.download(np.float32, n), -old)
    prog.run([x], [out])             # sees `new`
    assert np.array_equal(out.download(np.float32, n), -new)
    prog.close()
    x.close()
    out.close()


def test_async_run_reports_failure_on_wait(ctx):
    R, C = 16, 4
    pb = ProgramBuilder()
    sx, sy, sl = pb.input(R * C), pb.input(R, "i64"), pb.output(1)
    pb.index_ce(sx, sy, sl, R, C)
    prog = HipProgram(ctx, pb.image())
    x = ctx.upload(np.zeros(R * C, np.float32))
    y = np.zeros(R, np.int64)
    y[3] = 9
    yb = ctx.upload(y)
    loss = ctx.buffer(4)
    prog.run_async([x, yb], [loss])
    with pytest.raises(HipIndexError):
        prog.wait()
    prog.wait()  # nothing pending: returns
    yb.upload(np.zeros(R, np.int64))
    prog.run_async([x, yb], [loss])
    prog.run([x, yb], [loss])  # waits for the pending run first
    assert abs(loss.download(np.float32, 1)[0] - np.log(4.0)) < 1e-6
    prog.close()


def _batches(k, batch, fin, fout, loss, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(k):
        x = rng.standard_normal((batch, fin)).astype(np.float32)
        y = (rng.standard_normal((batch, fout)).astype(np.float32) if loss == "mse"
             else rng.integers(0, fout, batch).astype(np.int64))
        out.append((x, y))
    return out


def _bits(st):
    return [a.view(np.uint32).copy() for a in st.weights + st.biases + st.first + st.second]


@pytest.mark.parametrize("dims,loss,opt", [
    ([64, 128, 128, 16], "mse", Sgd(0.01, momentum=0.9)),
    ([96, 256, 10], "ce", Adam(1e-3)),
], ids=["mse-sgd", "ce-adam"])
def test_pipelined_training_matches_step_by_step(ctx, dims, loss, opt):
    spec = MlpSpec.chain(dims, hidden="relu", loss=loss)
    Ws, bs = init_parameters(spec, 3, "he_normal")
    batches = _batches(6, 512, dims[0], dims[-1], loss, 11)
    a = HipTrainingSession.open(ctx, spec, Ws, bs, opt, 512)
    want = [a.run(x, y).objective for x, y in batches]
    b = HipTrainingSession.open(ctx, spec, Ws, bs, opt, 512)
    got = [s.objective for s in b.run_pipelined(batches)]
    assert np.array_equal(np.array(got, np.float32).view(np.uint32),
                          np.array(want, np.float32).view(np.uint32))
    assert b.optimizer_steps == a.optimizer_steps == 6
    for u, v in zip(_bits(a.state()), _bits(b.state())):
        assert np.array_equal(u, v)
    a.close()
    b.close()


def test_pipelined_training_stops_at_a_failed_step(ctx):
    spec = MlpSpec.chain([4, 8, 1], hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    x = np.ones((8, 4), np.float32)
    good, bad = (x, np.zeros((8, 1), np.float32)), (x, np.full((8, 1), 3e38, np.float32))
    ref = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 8)
    ref.run(*good)
    ref.run(*good)
    s = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 8)
    with pytest.raises(HipArithmeticError):
        s.run_pipelined([good, good, bad, good])
    assert s.optimizer_steps == 2
    for u, v in zip(_bits(ref.state()), _bits(s.state())):
        assert np.array_equal(u, v)
    s.run(*good)  # the session stays usable
    assert s.optimizer_steps == 3
    ref.close()
    s.close()


def test_mismatched_batches_raise_and_change_nothing(ctx):
    spec = MlpSpec.chain([4, 8, 1], hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    x = np.ones((8, 4), np.float32)
    good = (x, np.zeros((8, 1), np.float32))
    s = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 8)
    s.run(*good)
    before = _bits(s.state())
    short = (x[:6], np.zeros((6, 1), np.float32))  # a short final batch
    wide = (np.ones((8, 5), np.float32), np.zeros((8, 1), np.float32))
    for bad in (short, wide):
        with pytest.raises(ValueError):
            s.run(*bad)
        with pytest.raises(ValueError):
            s.run_pipelined([good, bad, good])  # checked before the first run
    assert s.optimizer_steps == 1
    for u, v in zip(before, _bits(s.state())):
        assert np.array_equal(u, v)
    s.close()


def test_staging_failure_after_a_committed_run_keeps_that_run(ctx, monkeypatch):
    """The next batch's staging raises while step 1 is pending: step 1 still commits on the
    device, so the session must adopt its candidate set before the error propagates."""
    spec = MlpSpec.chain([4, 8, 1], hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    x = np.ones((8, 4), np.float32)
    good = (x, np.zeros((8, 1), np.float32))
    ref = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 8)
    ref.run(*good)
    s = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 8)
    s.run(*good)  # creates the session's batch buffers
    s._x2 = s.ctx.buffer(s._x.nbytes)
    s._y2 = s.ctx.buffer(s._y.nbytes)

    def refuse(*a, **k):
        raise RuntimeError("staging refused")

    monkeypatch.setattr(s._x2, "upload_staged", refuse)
    ref.run(*good)
    with pytest.raises(RuntimeError, match="staging refused"):
        s.run_pipelined([good, good])
    assert s.optimizer_steps == ref.optimizer_steps == 2
    for u, v in zip(_bits(ref.state()), _bits(s.state())):
        assert np.array_equal(u, v)
    s.run(*good)
    ref.run(*good)
    for u, v in zip(_bits(ref.state()), _bits(s.state())):
        assert np.array_equal(u, v)
    ref.close()
    s.close()
