"""The HIP backend through the engine composition: Engine.builder().takeOwnership(
HipBackendIntegration) -> prepare (PrepareContext -> analyze -> memory plan -> finalize ->
contribute / assemble) -> run (RunState with borrowed inputs and created outputs, canonical
big-endian publication). Results must equal the same partition run directly through the SPI
roles, bit for bit, also when several threads run one prepared execution at once."""
import threading

import numpy as np
import pytest

from synaptik_amd.backend import HipBackendIntegration
from synaptik_amd.engine import CallerInput, CreatedBuffer, Engine
from tests.partitions import mlp_train_partition, softmax_ce_partition

pytestmark = pytest.mark.gpu


def _decode(raw: bytes, d):
    be = {"FLOAT32": ">f4", "INT64": ">i8", "INT32": ">i4"}[d.dtype]
    return np.frombuffer(raw, be).astype(be[1:]).reshape(d.shape)


def _mlp_inputs(seed, B, I, H, O):
    rng = np.random.default_rng(seed)
    return {"x": rng.standard_normal((B, I)).astype(np.float32),
            "W1": (rng.standard_normal((H, I)) * np.sqrt(2 / I)).astype(np.float32),
            "b1": (rng.standard_normal(H) * 0.1).astype(np.float32),
            "W2": (rng.standard_normal((O, H)) * np.sqrt(2 / H)).astype(np.float32),
            "b2": (rng.standard_normal(O) * 0.1).astype(np.float32),
            "t": rng.standard_normal((B, O)).astype(np.float32)}


@pytest.fixture()
def engine():
    e = Engine.builder().take_ownership(HipBackendIntegration.open(0)).build()
    yield e
    e.close()


def test_engine_run_equals_the_direct_spi_run(engine):
    dims = (256, 64, 96, 10)
    part = mlp_train_partition(*dims)
    prepared = engine.prepare(part)
    plan = prepared.schedule.memory_plan
    assert [b.role for b in plan.buffers] == ["input"] * 6 + ["output"] * 7
    assert all(isinstance(p[0], CallerInput) for p, b in
               zip(prepared.schedule.buffer_preparations, plan.buffers) if b.role == "input")
    assert all(isinstance(p[0], CreatedBuffer) for p, b in
               zip(prepared.schedule.buffer_preparations, plan.buffers) if b.role == "output")
    values = _mlp_inputs(1, *dims)
    got = prepared.run(values)
    comp = engine.compositions()[0]
    direct = comp.integration.prepare(part)
    want = direct.run_values(values)
    for v in part.outputs:
        g = _decode(got[v], part.values[v])
        assert np.array_equal(g.view(np.uint32), np.asarray(want[v], np.float32).reshape(g.shape)
                              .view(np.uint32)), v
    direct.close()
    prepared.close()
    prepared.close()  # idempotent
    with pytest.raises(RuntimeError):
        prepared.run(values)


def test_concurrent_runs_of_one_prepared_execution_are_isolated(engine):
    R, C = 2048, 100
    part = softmax_ce_partition(R, C)
    prepared = engine.prepare(part)
    inputs = []
    for t in range(4):
        rng = np.random.default_rng(10 + t)
        inputs.append({"x": (rng.standard_normal((R, C)) * 3).astype(np.float32),
                       "g": rng.standard_normal((R, C)).astype(np.float32),
                       "labels": rng.integers(0, C, R).astype(np.int64)})
    want = [prepared.run(v) for v in inputs]
    got = [[None] * 5 for _ in inputs]
    barrier = threading.Barrier(4)
    errors = []

    def work(t):
        try:
            barrier.wait()
            for r in range(5):
                got[t][r] = prepared.run(inputs[t])
        except BaseException as e:  # noqa: BLE001 - re-raised below
            errors.append(e)

    ts = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for th in ts:
        th.start()
    for th in ts:
        th.join(120)
    assert not errors, errors
    for t in range(4):
        for r in range(5):
            assert got[t][r] == want[t], (t, r)
    prepared.close()


def test_second_integration_with_the_same_id_is_rejected_and_closed():
    first = HipBackendIntegration.open(0)
    second = HipBackendIntegration.open(0)
    builder = Engine.builder().take_ownership(first)
    with pytest.raises(ValueError, match="duplicate backend ID: hip"):
        builder.take_ownership(second)
    assert not second.context.handle  # ownership moved at entry: closed on rejection
    engine = builder.build()
    assert engine.compositions()[0].availability_snapshots()[0]["backend"] == "hip"
    engine.close()
    assert not first.context.handle
    with pytest.raises(RuntimeError):
        engine.prepare(mlp_train_partition(16, 8, 12, 4))


def test_traced_invocations_report_outcomes():
    """With a trace observer set, each bound run of a prepared executable emits its plan, timing
    and outcome; an out-of-range label yields FAILED with the native status code."""
    from synaptik_amd.trace import BackendInvocationOutcome, HipInvocationPlan, TraceOutcomeStatus
    integ = HipBackendIntegration.open(0)
    records = []
    integ.set_trace_observer(records.append)
    R, C = 64, 10
    exe = integ.prepare(softmax_ce_partition(R, C))
    rng = np.random.default_rng(0)
    vals = {"x": rng.standard_normal((R, C)).astype(np.float32),
            "g": rng.standard_normal((R, C)).astype(np.float32),
            "labels": rng.integers(0, C, R).astype(np.int64)}
    exe.run_values(vals)
    bad = dict(vals, labels=np.full(R, C + 1, np.int64))
    with pytest.raises(Exception):
        exe.run_values(bad)
    outcomes = [r for r in records if isinstance(r, BackendInvocationOutcome)]
    plans = [r for r in records if isinstance(r, HipInvocationPlan)]
    assert [o.status for o in outcomes] == [TraceOutcomeStatus.SUCCEEDED, TraceOutcomeStatus.FAILED]
    assert outcomes[1].native_status.code == 16
    assert plans[0].feed_slot_count == 3 and plans[0].aggregate_input_bytes == R * C * 8 + R * 8
    assert plans[0].aggregate_internal_bytes > 0
    exe.close()
    integ.close()
