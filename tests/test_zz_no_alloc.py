"""shk_hip_program_run_static, the entry point that allocates nothing: its per-run device memory
is the library's static per-device array. The bar is shk_hip_program_run's result on the same
inputs, bit for bit, over two calls in a row of which the second has a smaller input (the array
keeps the first call's contents), for programs that use the reduction scratch, the status word
and internal slots."""
import numpy as np
import pytest

from synaptik_amd.native import HipIndexError, HipInvalidArgument, HipProgram
from synaptik_amd.program import ProgramBuilder
from synaptik_amd.training import Adam, HipTrainingSession, MlpSpec, init_parameters, lower_forward

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _state_bits(st):
    return [_bits(a) for a in st.weights + st.biases + st.first + st.second]


def _session_pair(ctx, batch):
    spec = MlpSpec.chain([784, 1024, 1024, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 3, "he_normal")
    a = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), batch)
    b = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), batch)
    prog = b.program
    # every step of b runs through the no-allocation entry point
    prog.run = prog.run_static
    prog.run_bound = lambda bound: prog.run_static(list(bound.buffers[0]), list(bound.buffers[1]))
    return a, b


def test_training_steps_match_the_leased_run_big_then_small(ctx):
    rng = np.random.default_rng(1)
    for batch in (512, 96):  # the second call's program is smaller
        a, b = _session_pair(ctx, batch)
        for _ in range(2):
            x = rng.uniform(0, 1, (batch, 784)).astype(np.float32)
            y = rng.integers(0, 10, batch).astype(np.int64)
            oa = a.run(x, y).objective
            ob = b.run(x, y).objective
            assert _bits(np.float32(oa)) == _bits(np.float32(ob)), batch
            for u, v in zip(_state_bits(a.state()), _state_bits(b.state())):
                assert np.array_equal(u, v), batch
        a.close()
        b.close()


def _loss_program(R, C):
    pb = ProgramBuilder()
    x = pb.input(R * C)
    lab = pb.input(R, "i64")
    outs = [pb.output(1), pb.output(R * C), pb.output(1), pb.output(R)]
    pb.index_ce(x, lab, outs[0], R, C, grad=outs[1])
    pb.reduce_all(x, outs[2], R * C, "mean")
    pb.row_reduce(x, outs[3], R, C, "lse")
    return pb, outs


@pytest.mark.parametrize("shapes", [((4096, 1000), (300, 37))], ids=["big-then-small"])
def test_reduction_programs_match_the_leased_run(ctx, shapes):
    rng = np.random.default_rng(2)
    for R, C in shapes:
        pb, outs = _loss_program(R, C)
        prog = HipProgram(ctx, pb.image())
        x = ctx.upload((rng.standard_normal((R, C)) * 3).astype(np.float32))
        lab = ctx.upload(rng.integers(0, C, R).astype(np.int64))
        got, want = [], []
        for runner, dst in ((prog.run_static, got), (prog.run, want)):
            o = [ctx.buffer(s.nbytes) for s in outs]
            runner([x, lab], o)
            dst.extend(b.download(np.float32, s.count) for b, s in zip(o, outs))
        for g, w in zip(got, want):
            assert np.array_equal(_bits(g), _bits(w)), (R, C)
        prog.close()


def test_status_word_is_cleared_between_calls(ctx):
    """An out-of-range label fails one static call; the next call on clean labels succeeds and
    matches the leased run."""
    R, C = 1000, 10
    pb, outs = _loss_program(R, C)
    prog = HipProgram(ctx, pb.image())
    rng = np.random.default_rng(3)
    x = ctx.upload(rng.standard_normal((R, C)).astype(np.float32))
    bad = rng.integers(0, C, R).astype(np.int64)
    bad[5] = -2
    o = [ctx.buffer(s.nbytes) for s in outs]
    with pytest.raises(HipIndexError):
        prog.run_static([x, ctx.upload(bad)], o)
    good = ctx.upload(rng.integers(0, C, R).astype(np.int64))
    prog.run_static([x, good], o)
    w = [ctx.buffer(s.nbytes) for s in outs]
    prog.run([x, good], w)
    for g, v, s in zip(o, w, outs):
        assert np.array_equal(_bits(g.download(np.float32, s.count)),
                              _bits(v.download(np.float32, s.count)))
    prog.close()


def test_programs_beyond_the_static_array_are_refused(ctx):
    spec = MlpSpec.chain([4096, 4096, 4096], hidden="relu")
    prog = HipProgram(ctx, lower_forward(spec, 8192).image())
    assert prog.arena_bytes() > 64 << 20
    Ws, bs = init_parameters(spec, 0, "he_normal")
    ins = ([ctx.upload(w) for w in Ws] + [ctx.upload(b) for b in bs]
           + [ctx.buffer(8192 * 4096 * 4)])
    with pytest.raises(HipInvalidArgument, match="at most"):
        prog.run_static(ins, [ctx.buffer(8192 * 4096 * 4)])
    prog.close()


def test_calls_through_two_contexts_of_one_device_do_not_interfere():
    """Two contexts of device 0, each with a program of its own, call run_static from two threads
    at once. The calls share the device's array; the per-device lock serializes them, so every
    result equals that context's leased run bit for bit."""
    import threading

    from synaptik_amd.native import HipContext

    rng = np.random.default_rng(4)
    jobs = []
    for R, C in ((2048, 333), (1500, 64)):
        c = HipContext(0)
        pb, outs = _loss_program(R, C)
        prog = HipProgram(c, pb.image())
        x = c.upload((rng.standard_normal((R, C)) * 3).astype(np.float32))
        lab = c.upload(rng.integers(0, C, R).astype(np.int64))
        w = [c.buffer(s.nbytes) for s in outs]
        prog.run([x, lab], w)
        want = [b.download(np.float32, s.count) for b, s in zip(w, outs)]
        jobs.append(dict(ctx=c, prog=prog, ins=[x, lab], outs=outs, want=want, bad=[]))

    def work(j):
        o = [j["ctx"].buffer(s.nbytes) for s in j["outs"]]
        for it in range(25):
            j["prog"].run_static(j["ins"], o)
            for k, (b, s) in enumerate(zip(o, j["outs"])):
                if not np.array_equal(_bits(b.download(np.float32, s.count)), _bits(j["want"][k])):
                    j["bad"].append((it, k))

    threads = [threading.Thread(target=work, args=(j,)) for j in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for j in jobs:
        assert not j["bad"], j["bad"][:5]
        j["prog"].close()
        j["ctx"].close()
