"""The runtime's two-stream step schedule is race-free for every lowered program of the test
corpus: every pair of steps whose memory effects conflict (slots, the stream's reduction scratch,
the status word) is ordered by stream order, an event wait, or the final join (tests/plan_hazards.py
restates the effects from the kernels, independently of the runtime's own dependency model).
No device is needed: the plan comes from shk_hip_program_plan over the image."""
import itertools

import pytest

import synaptik_amd.training as training
from synaptik_amd.backend import HipPartitionPreparer
from synaptik_amd.native import program_plan
from synaptik_amd.program import OP_CE_HEAD, OP_OPTIMIZER, OP_STEP_COMMIT
from synaptik_amd.training import (Adam, AdamW, Dense, GradientMode, MlpSpec, Sgd,
                                   lower_dense_layer, lower_forward, lower_training_step)
from tests import plan_hazards as H
from tests.conftest import needs_fold, needs_two_streams

OPTS = [Sgd(0.05), Sgd(0.02, momentum=0.9, nesterov=True, weight_decay=0.01),
        Sgd(0.02, momentum=0.5, dampening=0.2), Adam(1e-3), AdamW(1e-3, 0.9, 0.999, 1e-8, 0.01)]
SPECS = [([24, 32, 32, 5], "relu", "ce", 128), ([784, 1024, 1024, 10], "relu", "ce", 1024),
         ([16, 64, 1], "tanh", "mse", 256), ([4096] * 6, "relu", "mse", 4096),
         ([256, 512, 512, 512, 256], "relu", "mse", 512), ([64, 256, 256, 16], "tanh", "mse", 512),
         ([32, 64, 8], "relu", "mse", 128), ([10, 7], None, "ce", 33), ([5, 3, 2], "sigmoid", "mse", 9),
         ([64, 48, 3], "tanh", "ce", 37)]
MODES = [(GradientMode.RESET_AND_STEP, False), (GradientMode.RESET_AND_STEP, True),
         (GradientMode.ACCUMULATE, False), (GradientMode.ACCUMULATE_AND_STEP, False)]


def _corpus():
    for fused in (True, False):
        old = training.FUSE_CE_HEAD
        training.FUSE_CE_HEAD = fused
        try:
            for (dims, act, loss, B), opt, (mode, clear) in itertools.product(SPECS, OPTS, MODES):
                if not fused and loss != "ce":
                    continue
                spec = MlpSpec.chain(dims, hidden=act, loss=loss)
                pb, _ = lower_training_step(spec, B, opt, mode=mode, clear_accumulator=clear)
                yield (f"train {dims} {loss} {type(opt).__name__} {mode} clear={clear} "
                       f"fused={fused}"), pb.image()
        finally:
            training.FUSE_CE_HEAD = old
    for dims, act, loss, B in SPECS:
        yield f"forward {dims}", lower_forward(MlpSpec.chain(dims, hidden=act, loss=loss), B).image()
    for args in [(8192, 1024, 1024, "relu", "in_out"), (64, 32, 32, "relu", "in_out"),
                 (100, 30, 20, "tanh", "out_in")]:
        yield f"dense {args}", lower_dense_layer(*args)[0].image()
    import tests.test_random_matmul_partitions_gpu as rm
    import tests.test_random_mlps_gpu as rmlp
    import tests.test_random_partitions_gpu as rp
    for seed in range(128):
        yield f"elementwise partition {seed}", HipPartitionPreparer().analyze(rp._graph(seed)[0]).plan
    for seed in range(64):
        yield f"matmul partition {seed}", HipPartitionPreparer().analyze(rm._graph(seed)[0]).plan
    for seed in range(64):
        dims, acts, loss, batch, opt, _odict, bias, _rng = rmlp._config(seed)
        spec = MlpSpec([Dense(a, b, act, bb) for a, b, act, bb in zip(dims, dims[1:], acts, bias)], loss)
        for mode in (GradientMode.RESET_AND_STEP, GradientMode.ACCUMULATE,
                     GradientMode.ACCUMULATE_AND_STEP):
            yield f"random mlp {seed} {mode}", lower_training_step(spec, batch, opt, mode=mode)[0].image()


@pytest.fixture(scope="module")
def corpus():
    return [(name, img, H.decode(img)) for name, img in _corpus()]


@needs_two_streams
def test_runtime_plan_orders_every_conflicting_pair(corpus):
    side = 0
    for name, img, steps in corpus:
        stream_of, wait_for, folded = program_plan(img)
        hazards = H.check_plan(steps, stream_of, wait_for, folded)
        assert not hazards, f"{name}: {[str(h) for h in hazards[:4]]}"
        side += any(stream_of)
    assert side > len(corpus) // 2  # the two-stream plan is really exercised


@needs_two_streams
@needs_fold
def test_folded_steps_have_no_event_edges(corpus):
    """Folded steps are never launched: no step may wait for them (a capture would wait on an
    event never recorded in it) and no later launched step may conflict with them. C3's loss MEAN
    is folded (its bias update, 2058 elements, is not: a pass over more than 1024 elements in
    one workgroup costs more than its own launch), and so is C1's 65-element bias update."""
    counts = {"mean": 0, "opt": 0}
    for name, img, steps in corpus:
        stream_of, wait_for, folded = program_plan(img)
        n = len(steps)
        launched = n - 1 if steps[-1].opcode == OP_STEP_COMMIT else n
        for kind, f in zip(("mean", "opt"), folded):
            if f < 0:
                continue
            counts[kind] += 1
            assert f not in wait_for and stream_of[f] == 0 and wait_for[f] == -1, name
            ef = H.effects(steps[f], 0)
            for st in steps[f + 1:launched]:
                if st.index in folded:
                    continue  # performed after it, in program order, by the same launch
                assert not H.conflict(ef, H.effects(st, stream_of[st.index])), name
    assert counts["mean"] > 0 and counts["opt"] > 0
    names = {name: program_plan(img)[2] for name, img, _ in corpus}
    c3 = names["train [784, 1024, 1024, 10] ce Adam reset_and_step clear=False fused=True"]
    assert c3[0] >= 0 and c3[1] < 0
    c1 = names["train [16, 64, 1] mse Sgd reset_and_step clear=False fused=True"]
    assert c1[1] >= 0


def test_check_rejects_a_plan_with_a_dropped_wait(corpus):
    """Every wait of the runtime's plans is needed (the planner skips a wait that an earlier wait
    of the same stream already covers): removing any one leaves a conflicting pair unordered, and
    the check names it."""
    tried = 0
    for name, img, steps in corpus[:120]:
        stream_of, wait_for, folded = program_plan(img)
        in_publication = set(folded) | {len(steps) - 1 if steps[-1].opcode == OP_STEP_COMMIT else -1}
        for j, w in enumerate(wait_for):
            if w < 0 or j in in_publication:  # never launched: its wait is unused
                continue
            cut = list(wait_for)
            cut[j] = -1
            assert H.check_plan(steps, stream_of, cut, folded), (name, j, w)
            tried += 1
    if tried == 0:
        pytest.skip("one-stream plans (SHK_HIP_CONCURRENT=0): no waits to drop")


def test_optimizer_status_reads_are_dependencies(corpus):
    """The optimizer's apply phase and accumulator commit / clear act only when the status word is
    clear. A planner that misses these reads (the runtime's model before they were added) puts
    the accumulator clear of RESET_AND_STEP-with-clear, and the commits of the accumulating
    modes, beside status-flagging steps; the check rejects those plans, and accepts the same
    greedy rule with the reads."""
    rejected = 0
    for name, img, steps in corpus:
        without = H.greedy_plan(steps, status_reads=False)
        hazards = H.check_plan(steps, *without)
        if hazards:
            rejected += 1
            assert all(steps[h.second].opcode == OP_OPTIMIZER and
                       (steps[h.second].iargs[0] in (4, 5) or steps[h.second].iargs[1] == 1)
                       for h in hazards), name
        assert not H.check_plan(steps, *H.greedy_plan(steps)), name
    assert rejected > 0


def test_critical_path_assignment_is_race_free_too(corpus):
    """A critical-path assignment (longest cost-weighted chain on the context stream, the rest
    beside it) with the same wait rule (the latest conflicting step of the other stream) is
    race-free on every program: which stream a step goes to cannot drop an edge."""
    for name, img, steps in corpus:
        stream_of, wait_for = H.critical_path_plan(steps)
        assert not H.check_plan(steps, stream_of, wait_for), name


def test_check_sees_scratch_and_status_conflicts():
    """Hand-made plans: two reductions sharing the context stream's scratch may not overlap, on
    different streams they may; a status OR beside the step commit is a hazard."""
    from synaptik_amd.program import ProgramBuilder
    pb = ProgramBuilder()
    a, b = pb.input(4096), pb.input(4096)
    o1, o2 = pb.output(1), pb.output(1)
    pb.reduce_all(a, o1, 4096, "sum")
    pb.reduce_all(b, o2, 4096, "sum")
    steps = H.decode(pb.image())
    assert not H.check_plan(steps, [0, 1], [-1, -1])        # own scratch each
    assert not H.check_plan(steps, [0, 0], [-1, -1])        # stream order
    # same scratch on one stream cannot be tested unordered; a cross-stream slot conflict can:
    pb = ProgramBuilder()
    a = pb.input(4096)
    t = pb.internal(4096)
    o = pb.output(1)
    pb.copy(a, t, 4096)
    pb.reduce_all(t, o, 4096, "sum")
    steps = H.decode(pb.image())
    assert H.check_plan(steps, [0, 1], [-1, -1])
    assert not H.check_plan(steps, [0, 1], [-1, 0])
    pb = ProgramBuilder()
    logits, lab, cnt = pb.input(64 * 10), pb.input(64, "i64"), pb.input(1, "i64", inout=True)
    loss = pb.output(1)
    pb.index_ce(logits, lab, loss, 64, 10)
    pb.fill(pb.internal(4), 4)
    pb.step_commit(cnt)
    steps = H.decode(pb.image())
    assert not H.check_plan(steps, [1, 0, 0], [-1, -1, -1])  # the commit runs after the join
