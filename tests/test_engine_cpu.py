"""Engine composition on the host (no device): Engine.builder().takeOwnership lifecycle rules
(Engine.java:83-213) and the schedule contribution's checks (PreparedScheduleContribution.java:
21-124, PreparedRepresentationPlan.java:35-100)."""
import pytest

from synaptik_amd.engine import (CallerInput, ContributionBuffer, ContributionWorkspace,
                                 CreatedBuffer, EngineBuilder, Engine, PreparedBuffer,
                                 PreparedMemoryPlan, PreparedSchedule,
                                 PreparedScheduleContribution, PreparedWorkspace)


class FakeProvider:
    def __init__(self, ident):
        self.ident = ident

    def backend_id(self):
        return self.ident


class FakeComposition:
    """An EngineBackendComposition that records its close calls."""

    def __init__(self, ident="hip", snapshot_id=None, fail=False):
        self.ident, self.snapshot_id, self.fail, self.closed = ident, snapshot_id or ident, fail, 0

    def backend_id(self):
        if self.fail:
            raise RuntimeError("interrogation failed")
        return self.ident

    def capability_providers(self):
        return (FakeProvider(self.ident),)

    def availability_snapshots(self):
        return ({"backend": self.snapshot_id},)

    def close(self):
        self.closed += 1


def test_take_ownership_and_build():
    a, b = FakeComposition("hip"), FakeComposition("cpu")
    builder = Engine.builder()
    assert builder.take_ownership(a) is builder
    builder.take_ownership(b)
    engine = builder.build()
    assert [c.backend_id() for c in engine.compositions()] == ["hip", "cpu"]
    with pytest.raises(RuntimeError, match="spent"):  # a spent builder rejects and closes
        c = FakeComposition("x")
        builder.take_ownership(c)
    assert c.closed == 1
    with pytest.raises(RuntimeError):
        builder.build()
    builder.close()  # closing a spent builder does nothing
    assert a.closed == b.closed == 0
    engine.close()
    engine.close()  # idempotent
    assert a.closed == b.closed == 1


def test_rejections_close_what_was_transferred():
    builder = EngineBuilder()
    first = FakeComposition("hip")
    builder.take_ownership(first)
    dup = FakeComposition("hip")
    with pytest.raises(ValueError, match="duplicate backend ID: hip"):
        builder.take_ownership(dup)
    assert dup.closed == 1 and first.closed == 0
    mismatch = FakeComposition("gpu", snapshot_id="other")
    with pytest.raises(ValueError, match="identities disagree"):
        builder.take_ownership(mismatch)
    assert mismatch.closed == 1
    failing = FakeComposition(fail=True)
    with pytest.raises(RuntimeError, match="interrogation"):
        builder.take_ownership(failing)
    assert failing.closed == 1
    with pytest.raises(TypeError):
        builder.take_ownership(None)
    builder.close()  # an open builder closes its entries
    assert first.closed == 1
    with pytest.raises(RuntimeError):
        builder.take_ownership(FakeComposition("late"))


def test_build_without_backends_fails_and_closes_the_builder():
    builder = EngineBuilder()
    with pytest.raises(ValueError, match="at least one backend"):
        builder.build()
    late = FakeComposition()
    with pytest.raises(RuntimeError):
        builder.take_ownership(late)
    assert late.closed == 1


def _plan():
    return PreparedMemoryPlan(
        (PreparedBuffer(0, ("x",), 64, 256, ("hip",), "input"),
         PreparedBuffer(1, ("y",), 64, 256, ("cpu", "hip"), "output")),
        (PreparedWorkspace(0, "hip", 1024, 256),))


def test_contribution_ownership_and_coordinates_are_checked():
    plan = _plan()
    ok = PreparedScheduleContribution(
        "hip", (ContributionBuffer(0, 0, CallerInput()),
                ContributionBuffer(1, 1, CreatedBuffer(lambda n, a: None))),
        (ContributionWorkspace(0, lambda n, a: None),), plan)
    assert len(ok.buffers) == 2
    with pytest.raises(ValueError, match="does not belong"):  # representation 0 of buffer 1 is cpu's
        PreparedScheduleContribution("hip", (ContributionBuffer(1, 0, CallerInput()),), (), plan)
    with pytest.raises(ValueError, match="does not belong"):  # no representation 2
        PreparedScheduleContribution("hip", (ContributionBuffer(1, 2, CallerInput()),), (), plan)
    with pytest.raises(ValueError, match="duplicates a buffer"):
        PreparedScheduleContribution("hip", (ContributionBuffer(0, 0, CallerInput()),
                                             ContributionBuffer(0, 0, CallerInput())), (), plan)
    with pytest.raises(ValueError, match="non-negative"):
        PreparedScheduleContribution("hip", (ContributionBuffer(0, -1, CallerInput()),), (), plan)
    with pytest.raises(ValueError, match="duplicates a workspace"):
        PreparedScheduleContribution("hip", (), (ContributionWorkspace(0, None),
                                                 ContributionWorkspace(0, None)), plan)
    with pytest.raises(ValueError, match="does not belong"):
        PreparedScheduleContribution("cpu", (), (ContributionWorkspace(0, None),), plan)
    with pytest.raises(TypeError):
        PreparedScheduleContribution("hip", (ContributionBuffer(0, 0, "caller"),), (), plan)


def test_schedule_needs_a_preparation_per_buffer_and_a_creator_per_workspace():
    plan = _plan()
    with pytest.raises(ValueError, match="bufferPreparations size"):
        PreparedSchedule(plan, ((CallerInput(),),), (None,), (), (), ())
    with pytest.raises(ValueError, match="workspaceCreators size"):
        PreparedSchedule(plan, ((CallerInput(),), (CallerInput(),)), (), (), (), ())
    with pytest.raises(ValueError, match="must not be empty"):
        PreparedSchedule(plan, ((CallerInput(),), ()), (None,), (), (), ())


class _FakeExecutable:
    def __init__(self, log):
        self.log = log

    def close(self):
        self.log.append("executable closed")


def _execution(log):
    from synaptik_amd.engine import PreparedExecution

    class Schedule:
        executables = (_FakeExecutable(log),)

    return PreparedExecution(FakeComposition(), Schedule(), None)


def test_close_waits_for_runs_in_flight_and_rejects_new_ones():
    """PreparedExecution.close during a run: the run finishes on open executables, close returns
    only after it, and later runs are rejected (IllegalStateException)."""
    import threading
    log = []
    pe = _execution(log)
    started, release = threading.Event(), threading.Event()

    def slow_run(inputs, maximum_bytes):
        started.set()
        release.wait(5)
        log.append("run finished")
        return {}

    pe._run = slow_run
    runner = threading.Thread(target=pe.run, args=({},))
    runner.start()
    assert started.wait(5)
    closer = threading.Thread(target=pe.close)
    closer.start()
    closer.join(0.2)
    assert closer.is_alive() and log == []  # waiting for the run
    with pytest.raises(RuntimeError, match="closed"):
        pe.run({})
    release.set()
    runner.join(5)
    closer.join(5)
    assert log == ["run finished", "executable closed"]
    pe.close()  # idempotent
    assert log == ["run finished", "executable closed"]


def test_engine_close_closes_prepared_executions_before_compositions():
    log = []
    comp = FakeComposition()
    comp.close = lambda: log.append("composition closed")
    engine = Engine([comp])
    engine._prepared.append(_execution(log))
    engine.close()
    assert log == ["executable closed", "composition closed"]
    with pytest.raises(RuntimeError, match="closed"):
        engine.prepare(None)
