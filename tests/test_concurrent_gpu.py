"""Two-stream step schedule (shk_hip_program_set_concurrent / _side_steps): steps that do not
depend on the tail of the main chain run on the context's second stream. The bar is the
one-stream order itself: every output and the whole training state must be bit-identical with
the schedule on and off, through graph replay and direct launches."""
import numpy as np
import pytest

from synaptik_amd.native import HipProgram
from synaptik_amd.training import (Adam, HipTrainingSession, MlpSpec, Sgd, init_parameters,
                                   lower_dense_layer)
from tests.conftest import needs_two_streams

pytestmark = pytest.mark.gpu


def _bits(st):
    return [a.view(np.uint32).copy() for a in st.weights + st.biases + st.first + st.second]


@needs_two_streams
@pytest.mark.parametrize("graphs", [True, False])
@pytest.mark.parametrize("dims,loss,opt", [
    ([784, 1024, 1024, 10], "ce", Adam(1e-3)),
    ([256, 512, 512, 512, 256], "mse", Sgd(0.01, momentum=0.9)),
], ids=["c3", "mlp-mse"])
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
            if concurrent:
                assert prog.side_steps() > 0
            prog.set_concurrent(concurrent)
            if not concurrent:
                assert prog.side_steps() == 0
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
