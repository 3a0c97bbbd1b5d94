"""Two-stream step schedule (shk_hip_program_set_concurrent / _side_steps): steps that do not
depend on the tail of the main chain run on the context's second stream. The bar is the
one-stream order itself: every output and the whole training state must be bit-identical with
the schedule on and off, through graph replay and direct launches."""
import numpy as np
import pytest

from synaptik_amd.native import HipIndexError, HipProgram
from synaptik_amd.program import ProgramBuilder
from synaptik_amd.training import (Adam, GradientMode, HipTrainingSession, MlpSpec, Sgd,
                                   init_parameters, lower_dense_layer)
from tests.conftest import needs_two_streams

pytestmark = pytest.mark.gpu


def _bits(st):
    return [a.view(np.uint32).copy() for a in st.weights + st.biases + st.first + st.second]


@needs_two_streams
@pytest.mark.parametrize("graphs", [True, False])
@pytest.mark.parametrize("dims,loss,opt", [
    ([784, 1024, 1024, 10], "ce", Adam(1e-3)),
    ([256, 512, 512, 512, 256], "mse", Sgd(0.01, momentum=0.9)),
    ([24, 32, 32, 5], "ce", Adam(1e-3)),
], ids=["c3", "mlp-mse", "small-fused-head"])
def test_training_state_identical_with_and_without_side_stream(ctx, dims, loss, opt, graphs):
    spec = MlpSpec.chain(dims, hidden="relu", loss=loss)
    Ws, bs = init_parameters(spec, 2, "he_normal")
    rng = np.random.default_rng(4)
    B = 512
    batches = [(rng.uniform(0, 1, (B, dims[0])).astype(np.float32),
                rng.integers(0, dims[-1], B).astype(np.int64) if loss == "ce"
                else rng.standard_normal((B, dims[-1])).astype(np.float32)) for _ in range(4)]
    sessions = []
    for concurrent in (True, False):
        s = HipTrainingSession.open(ctx, spec, Ws, bs, opt, B)
        for prog, _ in s._programs.values():
            prog.set_graph_mode(graphs)
            prog.set_concurrent(concurrent)
            assert (prog.side_steps() > 0) == concurrent
        objs = [s.run(x, y).objective for x, y in batches]
        sessions.append((s, objs))
    (a, oa), (b, ob) = sessions
    assert np.array_equal(np.array(oa, np.float32), np.array(ob, np.float32))
    for u, v in zip(_bits(a.state()), _bits(b.state())):
        assert np.array_equal(u, v)
    a.close()
    b.close()


def test_fused_layer_outputs_identical_with_and_without_side_stream(ctx):
    B, I, O = 2048, 512, 768
    pb, outs = lower_dense_layer(B, I, O, "relu", "in_out")
    rng = np.random.default_rng(8)
    ins = [ctx.upload(rng.standard_normal(n, dtype=np.float32)) for n in (B * I, I * O, O, B * O)]
    results = []
    for concurrent in (True, False):
        prog = HipProgram(ctx, pb.image())
        prog.set_concurrent(concurrent)
        obs = [ctx.buffer(s.nbytes) for s in outs]
        for _ in range(3):  # capture, then replays
            prog.run(ins, obs)
        results.append([o.download(np.uint32) for o in obs])
        prog.close()
    for u, v in zip(*results):
        assert np.array_equal(u, v)


@needs_two_streams
def test_small_fused_head_classifier_in_every_launch_form(ctx):
    """The 24->32->32->5 classifier with the fused head, through every gradient mode (including
    an accumulate run whose labels fail): two-stream graph replay, two-stream direct launches,
    one-stream replay and one-stream direct launches give bit-identical objectives, parameters,
    moments and accumulators after every run, with unrelated eager work between the runs."""
    spec = MlpSpec.chain([24, 32, 32, 5], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 7, "he_normal")
    B = 128
    rng = np.random.default_rng(23)
    modes = [GradientMode.RESET_AND_STEP, GradientMode.ACCUMULATE, GradientMode.ACCUMULATE,
             GradientMode.ACCUMULATE_AND_STEP, GradientMode.RESET_AND_STEP,
             GradientMode.ACCUMULATE, GradientMode.RESET_AND_STEP, GradientMode.RESET_AND_STEP]
    batches = []
    for i, m in enumerate(modes):
        x = rng.standard_normal((B, 24)).astype(np.float32)
        y = rng.integers(0, 5, B).astype(np.int64)
        if i == 2:
            y[77] = 5  # out of range: the accumulate run fails and must leave no trace
        batches.append((x, y, m))
    pb = ProgramBuilder()
    a = pb.input(4096)
    o = pb.output(1)
    pb.reduce_all(a, o, 4096, "sum")
    side = HipProgram(ctx, pb.image())
    sa, so = ctx.upload(np.ones(4096, np.float32)), ctx.buffer(4)
    forms = [(True, True), (True, False), (False, True), (False, False)]  # (two streams, graphs)
    sessions = [HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3), B) for _ in forms]
    for i, (x, y, m) in enumerate(batches):
        objs, states = [], []
        for (two, graphs), sess in zip(forms, sessions):
            sess._program(m, m == GradientMode.RESET_AND_STEP and sess.accumulated_gradient_runs > 0)
            for prog, _ in sess._programs.values():
                prog.set_graph_mode(graphs)
                prog.set_concurrent(two)
                if not two:
                    assert prog.side_steps() == 0
            if i == 2:
                with pytest.raises(HipIndexError):
                    sess.run(x, y, m)
            else:
                objs.append(np.float32(sess.run(x, y, m).objective).view(np.uint32))
            side.run([sa], [so])
            st = sess.state()
            states.append([u.view(np.uint32).copy() for u in
                           st.weights + st.biases + st.first + st.second + st.accumulators])
        print(f"small head run={i} mode={m} objectives={objs}", flush=True)
        assert len(set(int(v) for v in objs)) <= 1, i
        for other in states[1:]:
            assert len(other) == len(states[0])
            for u, v in zip(states[0], other):
                assert np.array_equal(u, v), i
    assert sessions[0].program.side_steps() > 0
    for sess in sessions:
        sess.close()
    side.close()
