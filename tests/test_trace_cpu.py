"""Trace payloads and the producer protocol (BackendInvocationOutcome.java, TraceNativeStatus,
MetalTraceProducer's disable-on-observer-failure rule), without a device."""
import pytest

from synaptik_amd.trace import (BackendInvocationOutcome, HipInvocationPlan, HipInvocationTiming,
                                HipTraceProducer, TracedRun, TraceNativeStatus,
                                TraceOutcomeStatus, TraceRouteKind)


def test_native_status_and_outcome_consistency():
    assert TraceNativeStatus.of(0).kind == "SUCCESS"
    assert TraceNativeStatus.of(5).kind == "RANGE_OUT_OF_BOUNDS"
    assert TraceNativeStatus.of(16) == TraceNativeStatus("UNKNOWN", 16)
    with pytest.raises(ValueError):
        TraceNativeStatus("SUCCESS", 3)
    with pytest.raises(ValueError):
        TraceNativeStatus("COPY_FAILED", 0)
    ok = TraceNativeStatus.of(0)
    BackendInvocationOutcome("hip", 0, 1, 2, TraceOutcomeStatus.SUCCEEDED,
                             TraceRouteKind.GRAPH_EXECUTABLE, ok)
    with pytest.raises(ValueError, match="SUCCEEDED requires"):
        BackendInvocationOutcome("hip", 0, 1, 2, TraceOutcomeStatus.SUCCEEDED,
                                 TraceRouteKind.GRAPH_EXECUTABLE, None)
    with pytest.raises(ValueError, match="FAILED forbids"):
        BackendInvocationOutcome("hip", 0, 1, 2, TraceOutcomeStatus.FAILED,
                                 TraceRouteKind.GRAPH_EXECUTABLE, ok)


class Failure(Exception):
    status = 11


def test_traced_runs_emit_plan_timing_and_outcome_with_fresh_ids():
    records = []
    p = HipTraceProducer(records.append, "hip", 3)
    u1, u2 = p.prepare_unit(), p.prepare_unit()
    assert (u1.prepared_unit_id, u2.prepared_unit_id) == (0, 1)
    TracedRun(p, u1, 2, 1, 1, 64, 32, 512)(lambda: None)

    def boom():
        raise Failure()

    with pytest.raises(Failure):
        TracedRun(p, u2, 2, 1, 1, 64, 32, 512)(boom)
    kinds = [type(r) for r in records]
    assert kinds == [HipInvocationPlan, HipInvocationTiming, BackendInvocationOutcome] * 2
    assert records[0].aggregate_internal_bytes == 512 and records[0].feed_slot_count == 2
    assert records[2].status is TraceOutcomeStatus.SUCCEEDED and records[2].device_id == 3
    assert records[5].status is TraceOutcomeStatus.FAILED
    assert records[5].native_status == TraceNativeStatus("EXECUTION_FAILED", 11)
    assert [r.invocation_id for r in records[::3]] == [0, 1]
    assert records[1].wall_ms >= 0.0


def test_an_observer_failure_disables_tracing_but_not_the_run():
    calls = []

    def bad(record):
        calls.append(record)
        raise RuntimeError("observer down")

    p = HipTraceProducer(bad)
    u = p.prepare_unit()
    ran = []
    TracedRun(p, u, 1, 1, 0, 4, 4, 0)(lambda: ran.append(1))
    assert ran == [1] and len(calls) == 1 and not p.enabled
    TracedRun(p, u, 1, 1, 0, 4, 4, 0)(lambda: ran.append(2))
    assert ran == [1, 2] and len(calls) == 1 and p.prepare_unit() is None
    other = HipTraceProducer(lambda r: None)
    with pytest.raises(ValueError, match="another producer"):
        other.begin_invocation(u)
