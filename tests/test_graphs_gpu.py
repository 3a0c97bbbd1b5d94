"""HIP-graph replay of programs must equal step-by-step launches on every replay, with eager work
and host synchronizations between replays (the runtime captures no memset nodes: the status word
is cleared by a fill kernel)."""
import numpy as np
import pytest

from synaptik_amd.native import HipProgram
from synaptik_amd.program import ProgramBuilder
from synaptik_amd.training import (Adam, GradientMode, HipTrainingSession, MlpSpec, Sgd,
                                   init_parameters, lower_training_step)
from tests.conftest import needs_graph_default

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("opt", [Sgd(0.05, momentum=0.9), Adam(1e-3)])
def test_graph_replay_matches_direct_launches(ctx, opt):
    spec = MlpSpec.chain([64, 256, 256, 16], hidden="tanh", loss="mse")
    Ws, bs = init_parameters(spec, 4, "xavier_uniform")
    graph = HipTrainingSession.open(ctx, spec, Ws, bs, opt, 512)
    eager = HipTrainingSession.open(ctx, spec, Ws, bs, opt, 512)
    for prog, _ in eager._programs.values():
        prog.set_graph_mode(False)
    eager.program.set_graph_mode(False)
    # unrelated eager work between replays
    pb = ProgramBuilder()
    a = pb.input(4096)
    o = pb.output(1)
    pb.reduce_all(a, o, 4096, "sum")
    side = HipProgram(ctx, pb.image())
    sa, so = ctx.upload(np.ones(4096, np.float32)), ctx.buffer(4)
    rng = np.random.default_rng(5)
    for step in range(6):
        x = rng.standard_normal((512, 64)).astype(np.float32)
        y = rng.standard_normal((512, 16)).astype(np.float32)
        g = graph.run(x, y)
        side.run([sa], [so])
        assert so.download()[0] == 4096.0
        e = eager.run(x, y)
        assert g.objective == e.objective
        sg, se = graph.state(), eager.state()
        for u, v in zip(sg.weights + sg.biases + sg.first + sg.second,
                        se.weights + se.biases + se.first + se.second):
            assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), step
    graph.close()
    eager.close()
    side.close()


def test_graph_replay_accumulation_modes(ctx):
    spec = MlpSpec.chain([32, 64, 8], hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, 6, "he_normal")
    sess = [HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.1, momentum=0.5), 128) for _ in range(2)]
    rng = np.random.default_rng(6)
    batches = [(rng.standard_normal((128, 32)).astype(np.float32),
                rng.standard_normal((128, 8)).astype(np.float32)) for _ in range(4)]
    modes = [GradientMode.ACCUMULATE, GradientMode.ACCUMULATE_AND_STEP, GradientMode.ACCUMULATE,
             GradientMode.RESET_AND_STEP]
    for i, (x, y) in enumerate(batches):
        for k, s in enumerate(sess):
            if k == 1:
                s._program(modes[i], modes[i] == GradientMode.RESET_AND_STEP)[0].set_graph_mode(False)
                s.program.set_graph_mode(False)
            s.run(x, y, modes[i])
    a, b = sess[0].state(), sess[1].state()
    for u, v in zip(a.weights + a.biases + a.first, b.weights + b.biases + b.first):
        assert np.array_equal(u, v)


@needs_graph_default
def test_default_launch_mode_follows_the_program(ctx):
    """Programs of large GEMMs only, and programs of at most five launched steps, launch step by
    step by default; any other program replays a graph. Either mode gives identical results."""
    from synaptik_amd.training import lower_dense_layer
    B, I, O = 1024, 512, 512  # every GEMM 2^28 multiply-adds
    pb, outs = lower_dense_layer(B, I, O, "relu", "in_out")
    progs = [HipProgram(ctx, pb.image()) for _ in range(2)]
    assert not progs[0].graph_mode()
    progs[1].set_graph_mode(True)
    assert progs[1].graph_mode()
    rng = np.random.default_rng(8)
    ins = [ctx.upload(rng.standard_normal(n, dtype=np.float32)) for n in (B * I, I * O, O, B * O)]
    res = []
    for p in progs:
        obs = [ctx.buffer(s.nbytes) for s in outs]
        for _ in range(3):
            p.run(ins, obs)
        res.append([o.download() for o in obs])
        p.close()
    for u, v in zip(*res):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
    small, _ = lower_dense_layer(64, 32, 32, "relu", "in_out")
    p = HipProgram(ctx, small.image())
    assert not p.graph_mode()  # three launched steps: direct launches cost less than a replay
    p.close()
    spec = MlpSpec.chain([32, 64, 64, 8], hidden="relu", loss="mse")
    pb, _ = lower_training_step(spec, 64, Sgd(0.1))
    p = HipProgram(ctx, pb.image())
    assert p.graph_mode()
    p.set_graph_mode(False)
    assert not p.graph_mode()
    p.close()
