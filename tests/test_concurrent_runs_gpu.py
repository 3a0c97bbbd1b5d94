"""Concurrent runs through the C ABI from several threads (Engine.java:480-507: "concurrent
calls have isolated state"; docs/backend-guide/writing-a-backend.md:140-142: per-run buffers
and workspaces belong to one RunState). Each run holds a per-run lease of the program (arena
with the internal slots, reduction scratch and status word); the bar is that every result is
bit-identical to the same runs made one after another on one thread."""
import threading

import numpy as np
import pytest

from synaptik_amd.native import HipArithmeticError, HipIndexError, HipProgram
from synaptik_amd.program import ProgramBuilder
from synaptik_amd.training import (Adam, HipTrainingSession, MlpSpec, Sgd, init_parameters,
                                   lower_forward)

pytestmark = pytest.mark.gpu

THREADS = 4
ROUNDS = 6


def _run_threads(fn, n=THREADS):
    """Runs fn(i) on n threads that start together; re-raises the first failure."""
    barrier = threading.Barrier(n)
    errors = []

    def body(i):
        try:
            barrier.wait()
            fn(i)
        except BaseException as e:  # noqa: BLE001 - reported below
            errors.append(e)

    ts = [threading.Thread(target=body, args=(i,)) for i in range(n)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(120)
    assert not any(t.is_alive() for t in ts), "a thread did not finish"
    if errors:
        raise errors[0]


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("graphs", [True, False])
def test_one_prepared_inference_program_from_many_threads(ctx, graphs):
    """A 3-layer inference program with internal activations, run by 4 threads on their own
    inputs and outputs, 6 rounds each: every output equals the sequential run of its input."""
    spec = MlpSpec.chain([512, 2048, 2048, 256], hidden="relu")
    Ws, bs = init_parameters(spec, 1, "he_normal")
    B = 1024
    prog = HipProgram(ctx, lower_forward(spec, B).image())
    prog.set_graph_mode(graphs)
    params = [ctx.upload(w) for w in Ws] + [ctx.upload(b) for b in bs]
    rng = np.random.default_rng(5)
    xs = [[ctx.upload(rng.standard_normal((B, 512)).astype(np.float32)) for _ in range(ROUNDS)]
          for _ in range(THREADS)]
    want = []
    for t in range(THREADS):
        row = []
        for r in range(ROUNDS):
            out = ctx.buffer(B * 256 * 4)
            prog.run(params + [xs[t][r]], [out])
            row.append(out.download(np.float32, B * 256))
        want.append(row)
    outs = [[ctx.buffer(B * 256 * 4) for _ in range(ROUNDS)] for _ in range(THREADS)]

    def work(t):
        for r in range(ROUNDS):
            prog.run(params + [xs[t][r]], [outs[t][r]])

    _run_threads(work)
    for t in range(THREADS):
        for r in range(ROUNDS):
            assert np.array_equal(_bits(outs[t][r].download(np.float32, B * 256)),
                                  _bits(want[t][r])), (t, r)
    assert 1 <= prog.lease_count() <= 4
    prog.close()


def _loss_program(R, C):
    """Cross-entropy over logits with its gradient, plus a whole-tensor MEAN of the logits:
    both use the lease's reduction scratch, the loss also its status word (label bounds)."""
    pb = ProgramBuilder()
    x = pb.input(R * C)
    lab = pb.input(R, "i64")
    loss = pb.output(1)
    grad = pb.output(R * C)
    mean = pb.output(1)
    pb.index_ce(x, lab, loss, R, C, grad=grad)
    pb.reduce_all(x, mean, R * C, "mean")
    return pb, (loss, grad, mean)


def test_reduction_scratch_and_status_are_per_run(ctx):
    """Threads run one loss program; one thread's labels are out of range on odd rounds. Only
    that thread's runs fail (INDEX_OUT_OF_BOUNDS from its own status word); every other result
    equals the sequential one bit for bit."""
    R, C = 4096, 1000
    pb, slots = _loss_program(R, C)
    prog = HipProgram(ctx, pb.image())
    rng = np.random.default_rng(9)
    xs = [ctx.upload((rng.standard_normal((R, C)) * 3).astype(np.float32)) for _ in range(THREADS)]
    good = [ctx.upload(rng.integers(0, C, R).astype(np.int64)) for _ in range(THREADS)]
    bad_labels = rng.integers(0, C, R).astype(np.int64)
    bad_labels[17] = C + 3
    bad = ctx.upload(bad_labels)

    def outputs():
        return [ctx.buffer(s.nbytes) for s in slots]

    def read(o):
        return [b.download(np.float32, s.count) for b, s in zip(o, slots)]

    want = []
    for t in range(THREADS):
        o = outputs()
        prog.run([xs[t], good[t]], o)
        want.append(read(o))
    results = [[None] * ROUNDS for _ in range(THREADS)]
    failures = [[False] * ROUNDS for _ in range(THREADS)]

    def work(t):
        for r in range(ROUNDS):
            o = outputs()
            try:
                prog.run([xs[t], bad if (t == 0 and r % 2 == 1) else good[t]], o)
                results[t][r] = read(o)
            except HipIndexError:
                failures[t][r] = True

    _run_threads(work)
    for t in range(THREADS):
        for r in range(ROUNDS):
            expect_fail = t == 0 and r % 2 == 1
            assert failures[t][r] == expect_fail, (t, r)
            if not expect_fail:
                for g, w in zip(results[t][r], want[t]):
                    assert np.array_equal(_bits(g), _bits(w)), (t, r)
    prog.close()


def test_two_programs_on_one_context_concurrently(ctx):
    """A training session (two-stream schedule, HIP graphs, fused optimizer) steps on one
    thread while an inference program of another network runs on a second thread: the
    training state and every inference output equal those of running them one after another."""
    spec = MlpSpec.chain([784, 1024, 1024, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 2, "he_normal")
    rng = np.random.default_rng(4)
    batches = [(rng.uniform(0, 1, (512, 784)).astype(np.float32),
                rng.integers(0, 10, 512).astype(np.int64)) for _ in range(8)]
    ispec = MlpSpec.chain([256, 1024, 64], hidden="tanh")
    iW, ib = init_parameters(ispec, 3, "xavier_uniform")
    iprog = HipProgram(ctx, lower_forward(ispec, 2048).image())
    iparams = [ctx.upload(w) for w in iW] + [ctx.upload(b) for b in ib]
    ixs = [ctx.upload(rng.standard_normal((2048, 256)).astype(np.float32)) for _ in range(8)]

    seq = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), 512)
    seq_obj = [seq.run(x, y).objective for x, y in batches]
    seq_state = seq.state()
    seq.close()
    iwant = []
    for x in ixs:
        o = ctx.buffer(2048 * 64 * 4)
        iprog.run(iparams + [x], [o])
        iwant.append(o.download(np.float32, 2048 * 64))

    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), 512)
    got_obj = []
    iout = [ctx.buffer(2048 * 64 * 4) for _ in ixs]

    def work(t):
        if t == 0:
            for x, y in batches:
                got_obj.append(sess.run(x, y).objective)
        else:
            for _ in range(3):
                for x, o in zip(ixs, iout):
                    iprog.run(iparams + [x], [o])

    _run_threads(work, 2)
    st = sess.state()
    assert np.array_equal(np.array(got_obj, np.float32).view(np.uint32),
                          np.array(seq_obj, np.float32).view(np.uint32))
    for a, b in zip(st.weights + st.biases + st.first + st.second,
                    seq_state.weights + seq_state.biases + seq_state.first + seq_state.second):
        assert np.array_equal(_bits(a), _bits(b))
    for o, w in zip(iout, iwant):
        assert np.array_equal(_bits(o.download(np.float32, 2048 * 64)), _bits(w))
    sess.close()
    iprog.close()


def test_failed_step_on_one_thread_leaves_other_sessions_untouched(ctx):
    """Two sessions of one network step concurrently; one of them is driven into a non-finite
    update (ARITHMETIC, nothing committed). The other's trajectory equals its sequential one."""
    spec = MlpSpec.chain([4, 64, 1], hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 0, "he_normal")
    x = np.ones((64, 4), np.float32)
    y = np.zeros((64, 1), np.float32)
    huge = np.full((64, 1), 3e38, np.float32)
    ref = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 64)
    want = [ref.run(x, y).objective for _ in range(10)]
    want_state = ref.state()
    ref.close()
    a = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 64)
    b = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.9), 64)
    got, failed = [], []

    def work(t):
        if t == 0:
            for _ in range(10):
                got.append(a.run(x, y).objective)
        else:
            for _ in range(10):
                try:
                    b.run(x, huge)
                except HipArithmeticError:
                    failed.append(True)

    _run_threads(work, 2)
    assert got == want and len(failed) == 10 and b.optimizer_steps == 0
    st = a.state()
    for u, v in zip(st.weights + st.biases + st.first, want_state.weights + want_state.biases
                    + want_state.first):
        assert np.array_equal(_bits(u), _bits(v))
    a.close()
    b.close()
