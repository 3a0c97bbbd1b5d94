"""Engine composition of the HIP backend: the host-side mirror of how the reference's Engine takes
ownership of a backend integration and prepares and runs partitions through it.

Reference shapes mirrored here (names kept, Java types as dataclasses):
  * Engine.builder().takeOwnership(integration).build() (modules/engine/.../Engine.java:83-213):
    ownership of the integration moves at call entry; a rejected registration (spent or closed
    builder, duplicate backend id, failing interrogation) closes what was transferred; build()
    needs at least one backend and spends the builder; closing an open builder closes its
    entries.
  * EngineBackendComposition (EngineBackendComposition.java:25-167), implemented like
    MetalEngineBackendComposition.java:24-178 by HipEngineBackendComposition: capability
    providers, availability snapshots, partition preparation, schedule contributor and
    assembler, transfers to a CPU composition, borrow of caller host storage, canonical
    publication, close.
  * PrepareContext (modules/prepare/.../analysis/PrepareContext.java:760-830): the planned
    partition, its nodes, graph values, logical memory requirements, constants and the backend's
    own inputs, projected from a compiled graph for one partition.
  * PreparedMemoryPlan / PreparedScheduleContext / PreparedScheduleContribution with
    CallerInput / CreatedBuffer / InitializedBuffer preparations and workspace creators
    (PreparedScheduleContribution.java:21-124, runtime/resource/PreparedRepresentationPlan.java
    :100-210), with the contribution's ownership and coordinate checks.
  * Per-run ownership (docs/backend-guide/writing-a-backend.md:140-142; Engine.java:480-507):
    a run creates a RunState holding its own created buffers (the published outputs) and the
    borrowed inputs; the prepared executable and its program are immutable and shared, and the
    program's per-run device state lives in the native per-run leases. Concurrent runs of one
    prepared execution are therefore isolated.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass, field
from typing import Callable, Optional, Sequence

import numpy as np

from .backend import (BACKEND_ID, STORAGE_WIDTH, CpuHipPreparedBufferTransfer,
                      HipBackendIntegration, HipCapabilityProvider, HipPartitionFinalizer,
                      HipPartitionPreparer, HipPreparedExecutable, OperationCapabilityQuery,
                      Partition, TensorDescriptor, UnsupportedPartition)
from .native import HipBuffer

ALIGNMENT = 256


# ---- the prepare-side records ----
@dataclass(frozen=True)
class GraphValue:
    id: str
    descriptor: TensorDescriptor


@dataclass(frozen=True)
class LogicalMemoryRequirement:
    value_id: str
    byte_size: int
    alignment: int = ALIGNMENT


@dataclass(frozen=True)
class PlannedPartition:
    index: int
    owner: str


def _byte_size(d: TensorDescriptor) -> int:
    return d.count * STORAGE_WIDTH[d.dtype]


@dataclass(frozen=True)
class PrepareContext:
    """What a partition preparer receives: one planned partition of a compiled graph."""
    partition: PlannedPartition
    nodes: tuple
    values: tuple                # GraphValue per value the partition reads or writes
    memory_requirements: tuple   # LogicalMemoryRequirement per value
    constants: dict
    backend_inputs: object
    graph: Partition             # the partition's node-list form the lowering consumes

    @staticmethod
    def project(graph: Partition, partition: PlannedPartition, backend_inputs) -> "PrepareContext":
        """GraphPreparation.project analogue: the partition's values, nodes and requirements."""
        values = tuple(GraphValue(v, d) for v, d in graph.values.items())
        reqs = tuple(LogicalMemoryRequirement(v, _byte_size(d)) for v, d in graph.values.items())
        return PrepareContext(partition, tuple(graph.nodes), values, reqs, {}, backend_inputs,
                              graph)


@dataclass(frozen=True)
class PreparedBuffer:
    """One prepared buffer of the memory plan: the values it holds, its size and alignment, and
    the backends owning each of its representations."""
    index: int
    value_ids: tuple
    byte_size: int
    alignment: int
    representation_owners: tuple
    role: str  # "input" (caller-bound) or "output" (published)


@dataclass(frozen=True)
class PreparedWorkspace:
    index: int
    owner: str
    byte_size: int
    alignment: int


@dataclass(frozen=True)
class PreparedMemoryPlan:
    buffers: tuple
    workspaces: tuple


@dataclass(frozen=True)
class CallerInput:
    """The representation is the caller's bound input for the run."""


@dataclass(frozen=True)
class CreatedBuffer:
    """The representation is created for each run by `creator(byte_size, alignment)`."""
    creator: Callable


@dataclass(frozen=True)
class InitializedBuffer:
    """Created by `creator` and initialized by the preparation before first use."""
    creator: Callable


@dataclass(frozen=True)
class ContributionBuffer:
    buffer_index: int
    representation_index: int
    preparation: object


@dataclass(frozen=True)
class ContributionWorkspace:
    workspace_index: int
    creator: Callable


@dataclass(frozen=True)
class PreparedScheduleContribution:
    """A backend's buffer preparations and workspace creators for the representations it owns
    (PreparedScheduleContribution.java:21-124)."""
    owner: str
    buffers: tuple
    workspaces: tuple
    memory_plan: PreparedMemoryPlan

    def __post_init__(self):
        seen = set()
        for i, b in enumerate(self.buffers):
            if not isinstance(b.preparation, (CallerInput, CreatedBuffer, InitializedBuffer)):
                raise TypeError(f"buffers[{i}] has no buffer preparation")
            if b.representation_index < 0:
                raise ValueError("representationIndex must be non-negative")
            owners = self.memory_plan.buffers[b.buffer_index].representation_owners
            if b.representation_index >= len(owners) or owners[b.representation_index] != self.owner:
                raise ValueError(f"buffers[{i}] does not belong to contribution owner")
            key = (b.buffer_index, b.representation_index)
            if key in seen:
                raise ValueError(f"buffers[{i}] duplicates a buffer representation coordinate")
            seen.add(key)
        ws = set()
        for i, w in enumerate(self.workspaces):
            if self.memory_plan.workspaces[w.workspace_index].owner != self.owner:
                raise ValueError(f"workspaces[{i}] does not belong to contribution owner")
            if w.workspace_index in ws:
                raise ValueError(f"workspaces[{i}] duplicates a workspace coordinate")
            ws.add(w.workspace_index)


@dataclass(frozen=True)
class PreparedScheduleContext:
    planned_partitions: tuple
    graph_values: tuple
    bindable_input_value_ids: tuple
    publication_value_ids: tuple
    memory_plan: PreparedMemoryPlan
    executables: tuple


@dataclass(frozen=True)
class PreparedSchedule:
    """The assembled schedule: one preparation list per buffer, a creator per workspace, and the
    executables in partition order (PreparedRepresentationPlan.java:35-100)."""
    memory_plan: PreparedMemoryPlan
    buffer_preparations: tuple
    workspace_creators: tuple
    executables: tuple
    input_value_ids: tuple
    publication_value_ids: tuple

    def __post_init__(self):
        if len(self.buffer_preparations) != len(self.memory_plan.buffers):
            raise ValueError("bufferPreparations size must equal prepared buffer count")
        if len(self.workspace_creators) != len(self.memory_plan.workspaces):
            raise ValueError("workspaceCreators size must equal prepared workspace count")
        for i, preps in enumerate(self.buffer_preparations):
            if not preps:
                raise ValueError(f"bufferPreparations[{i}] must not be empty")


# ---- the HIP roles the composition publishes ----
@dataclass(frozen=True)
class HipBackendInputs:
    """The backend's own preparation inputs (the Metal analogue carries tuning): the device
    facts the lowering could consult."""
    device: dict


@dataclass(frozen=True)
class PartitionPreparation:
    preparer: HipPartitionPreparer
    finalizer: HipPartitionFinalizer
    backend_inputs: HipBackendInputs


class HipScheduleContributor:
    """PreparedScheduleContributor: caller inputs stay CallerInput; every published value gets a
    CreatedBuffer whose creator allocates a device buffer of this integration per run. The HIP
    program needs no Engine workspace: its per-run arena is the program's native lease."""

    def __init__(self, integration: HipBackendIntegration):
        self.integration = integration

    def backend_id(self) -> str:
        return BACKEND_ID

    def _create(self, byte_size: int, alignment: int) -> HipBuffer:
        if alignment <= 0 or alignment & (alignment - 1) or alignment > ALIGNMENT:
            raise ValueError(f"unsupported buffer alignment {alignment}")
        return self.integration.context.buffer(max(int(byte_size), 4))

    def contribute(self, context: PreparedScheduleContext) -> PreparedScheduleContribution:
        buffers = []
        for b in context.memory_plan.buffers:
            for r, owner in enumerate(b.representation_owners):
                if owner != BACKEND_ID:
                    continue
                prep = CallerInput() if b.role == "input" else CreatedBuffer(self._create)
                buffers.append(ContributionBuffer(b.index, r, prep))
        return PreparedScheduleContribution(BACKEND_ID, tuple(buffers), (), context.memory_plan)


class HipScheduleAssembler:
    """PreparedScheduleAssembler for a context whose partitions all belong to the HIP backend."""

    def __init__(self, contributor: HipScheduleContributor):
        self.contributor = contributor

    def assemble(self, context: PreparedScheduleContext) -> PreparedSchedule:
        contribution = self.contributor.contribute(context)
        preps = [[] for _ in context.memory_plan.buffers]
        for b in contribution.buffers:
            lst = preps[b.buffer_index]
            while len(lst) <= b.representation_index:
                lst.append(None)
            lst[b.representation_index] = b.preparation
        creators = [None] * len(context.memory_plan.workspaces)
        for w in contribution.workspaces:
            creators[w.workspace_index] = w.creator
        return PreparedSchedule(context.memory_plan, tuple(tuple(p) for p in preps),
                                tuple(creators), context.executables,
                                context.bindable_input_value_ids,
                                context.publication_value_ids)

    def producerless_published_value(self, *a, **k):
        raise ValueError("schedule assembler does not support producerless published values")


class HipEngineBackendComposition:
    """EngineBackendComposition of the HIP integration (MetalEngineBackendComposition.java:24-178)."""

    def __init__(self, integration: HipBackendIntegration):
        if integration is None:
            raise TypeError("integration")
        self.integration = integration
        self._providers = (integration.capability_provider,)
        self._snapshots = (integration.availability_snapshot(),)
        self._contributor = HipScheduleContributor(integration)
        self._assembler = HipScheduleAssembler(self._contributor)
        self._preparation = PartitionPreparation(integration.preparer, integration.finalizer,
                                                 HipBackendInputs(self._snapshots[0]["device"]))

    def backend_id(self) -> str:
        return BACKEND_ID

    def capability_providers(self) -> tuple:
        return self._providers

    def availability_snapshots(self) -> tuple:
        return self._snapshots

    def partition_preparation(self) -> PartitionPreparation:
        return self._preparation

    def schedule_contributor(self) -> HipScheduleContributor:
        return self._contributor

    def schedule_assembler(self) -> HipScheduleAssembler:
        return self._assembler

    def supports_producerless_published_values(self) -> bool:
        return False

    def supports_transfer_to(self, destination, descriptor: TensorDescriptor) -> bool:
        if destination is None:
            raise TypeError("destination")
        return (getattr(destination, "backend_id", lambda: None)() == "cpu"
                and CpuHipPreparedBufferTransfer.supports(descriptor))

    def prepare_transfer_to(self, destination, memory_plan: PreparedMemoryPlan, buffer_index: int,
                            source_representation_index: int,
                            destination_representation_index: int,
                            descriptor: TensorDescriptor):
        if getattr(destination, "backend_id", lambda: None)() != "cpu":
            raise ValueError("HIP transfer destination is not the registered CPU adapter")
        return CpuHipPreparedBufferTransfer.hip_to_cpu(
            self.integration, memory_plan.buffers[buffer_index].byte_size, descriptor)

    def borrow(self, dtype: str, storage: np.ndarray) -> HipBuffer:
        return self.integration.borrow(dtype, storage)

    def copy_to_canonical_host_bytes(self, representation, descriptor, maximum_bytes: int):
        return self.integration.copy_to_canonical_host_bytes(representation, descriptor,
                                                             maximum_bytes)

    def close(self) -> None:
        self.integration.close()


# ---- preparation and runs ----
class RunState:
    """The buffers one run owns: its created representations (released when the run's results
    have been published) and its borrowed inputs."""

    def __init__(self):
        self.created: list[HipBuffer] = []
        self.borrowed: list[HipBuffer] = []

    def close(self):
        for b in self.created + self.borrowed:
            b.close()
        self.created.clear()
        self.borrowed.clear()


class PreparedExecution:
    """A prepared graph: the assembled schedule, its executables (immutable, shared by every
    run) and the compositions that own them. close() releases the prepared resources once: runs
    that start after it has begun are rejected, and it waits for the runs in flight to finish
    before the executables are closed."""

    def __init__(self, composition: HipEngineBackendComposition, schedule: PreparedSchedule,
                 graph: Partition):
        self.composition = composition
        self.schedule = schedule
        self.graph = graph
        self._lock = threading.Lock()
        self._idle = threading.Condition(self._lock)
        self._in_flight = 0
        self._closed = False

    def _enter(self):
        with self._lock:
            if self._closed:
                raise RuntimeError("prepared execution is closed")  # IllegalStateException
            self._in_flight += 1

    def _leave(self):
        with self._lock:
            self._in_flight -= 1
            if self._in_flight == 0:
                self._idle.notify_all()

    def run(self, inputs: dict, maximum_bytes: int = 1 << 40) -> dict:
        """One run: borrows every caller input, creates the published buffers, executes the
        bound invocation synchronously and returns each publication as canonical big-endian
        bytes (HostTensorValue.java:18). The per-run buffers are released before returning."""
        self._enter()
        try:
            return self._run(inputs, maximum_bytes)
        finally:
            self._leave()

    def _run(self, inputs: dict, maximum_bytes: int) -> dict:
        exe: HipPreparedExecutable = self.schedule.executables[0]
        plan = self.schedule.memory_plan
        state = RunState()
        try:
            bound_inputs = {}
            for b, preps in zip(plan.buffers, self.schedule.buffer_preparations):
                (vid,) = b.value_ids
                if isinstance(preps[0], CallerInput):
                    if vid not in inputs:
                        raise ValueError(f"missing bound input {vid}")
                    d = self.graph.values[vid]
                    host = np.asarray(inputs[vid])
                    want = {"FLOAT32": np.float32, "INT32": np.int32, "INT64": np.int64}[d.dtype]
                    if host.dtype != want or host.size != d.count:
                        raise ValueError(f"input {vid} does not match its descriptor {d}")
                    buf = self.composition.borrow(d.dtype, host)
                    state.borrowed.append(buf)
                    bound_inputs[vid] = buf
            outputs = []
            for b, preps in zip(plan.buffers, self.schedule.buffer_preparations):
                if b.role == "output":
                    buf = preps[0].creator(b.byte_size, b.alignment)
                    state.created.append(buf)
                    outputs.append(buf)
            outs = exe.bind(bound_inputs, outputs).execute()
            result = {}
            for vid, buf in zip(self.schedule.publication_value_ids, outs):
                result[vid] = bytes(self.composition.copy_to_canonical_host_bytes(
                    buf, self.graph.values[vid], maximum_bytes))
            return result
        finally:
            state.close()

    def close(self) -> None:
        with self._lock:
            if self._closed:
                return
            self._closed = True
            while self._in_flight:
                self._idle.wait()
        for exe in self.schedule.executables:
            exe.close()


class Engine:
    """Owns registered backend compositions and prepares / runs graphs through them."""

    def __init__(self, compositions: Sequence[HipEngineBackendComposition]):
        self._compositions = list(compositions)
        self._lock = threading.Lock()
        self._closed = False
        self._prepared: list[PreparedExecution] = []  # closed before the compositions

    @staticmethod
    def builder() -> "EngineBuilder":
        return EngineBuilder()

    def compositions(self) -> tuple:
        return tuple(self._compositions)

    def _owner_of(self, graph: Partition) -> HipEngineBackendComposition:
        for comp in self._compositions:
            providers = comp.capability_providers()
            ok = True
            for n in graph.nodes:
                q = OperationCapabilityQuery(n.kind, tuple(graph.values[v] for v in n.inputs),
                                             (graph.values[n.output],),
                                             tuple(sorted(n.attrs.items())))
                if not any(p.supports(q) for p in providers):
                    ok = False
                    break
            if ok:
                return comp
        raise UnsupportedPartition("no registered backend supports every node of the partition")

    def prepare(self, graph: Partition) -> PreparedExecution:
        """Plans the graph as one partition owned by the backend that supports all its nodes,
        then analyze -> memory plan -> finalize -> contribute / assemble."""
        with self._lock:
            if self._closed:
                raise RuntimeError("engine is closed")
        comp = self._owner_of(graph)
        prep = comp.partition_preparation()
        planned = PlannedPartition(0, comp.backend_id())
        context = PrepareContext.project(graph, planned, prep.backend_inputs)
        analysis = prep.preparer.analyze(context)
        buffers = []
        for v in graph.inputs:
            buffers.append(PreparedBuffer(len(buffers), (v,), _byte_size(graph.values[v]),
                                          ALIGNMENT, (comp.backend_id(),), "input"))
        for v in graph.outputs:
            buffers.append(PreparedBuffer(len(buffers), (v,), _byte_size(graph.values[v]),
                                          ALIGNMENT, (comp.backend_id(),), "output"))
        plan = PreparedMemoryPlan(tuple(buffers), ())
        exe = prep.finalizer.finalize_partition(analysis)
        try:
            sctx = PreparedScheduleContext((planned,), context.values, tuple(graph.inputs),
                                           tuple(graph.outputs), plan, (exe,))
            schedule = comp.schedule_assembler().assemble(sctx)
        except BaseException:
            exe.close()  # the finalizer's acquisitions roll back on failure
            raise
        execution = PreparedExecution(comp, schedule, graph)
        with self._lock:
            if not self._closed:
                self._prepared.append(execution)
                return execution
        execution.close()  # the engine closed while this graph was being prepared
        raise RuntimeError("engine is closed")

    def close(self) -> None:
        """Closes every prepared execution (waiting for its runs in flight), then every
        composition; each is closed even when an earlier one fails, and the first failure is
        raised."""
        with self._lock:
            if self._closed:
                return
            self._closed = True
            prepared, self._prepared = self._prepared, []
        errors = []
        for execution in prepared:
            try:
                execution.close()
            except Exception as e:  # noqa: BLE001
                errors.append(e)
        for comp in self._compositions:
            try:
                comp.close()
            except Exception as e:  # noqa: BLE001 - every entry is closed, then reported
                errors.append(e)
        if errors:
            raise errors[0]


class EngineBuilder:
    """Engine.Builder (Engine.java:83-213): takeOwnership / build / close with its states."""

    def __init__(self):
        self._entries: list = []
        self._state = "OPEN"
        self._lock = threading.Lock()

    def take_ownership(self, integration) -> "EngineBuilder":
        """Ownership moves at call entry: on any rejection the transferred integration (or the
        composition made from it) is closed before the failure propagates."""
        if integration is None:
            raise TypeError("integration")
        with self._lock:
            entry = None
            try:
                if self._state != "OPEN":
                    raise RuntimeError("engine builder is spent or closed")  # IllegalStateException
                if isinstance(integration, HipBackendIntegration):
                    entry = HipEngineBackendComposition(integration)
                else:
                    entry = integration  # an EngineBackendComposition directly
                ident = entry.backend_id()
                providers = entry.capability_providers()
                snapshots = entry.availability_snapshots()
                for p in providers:
                    if p.backend_id() != ident:
                        raise ValueError("provider and availability identities disagree")
                for s in snapshots:
                    if s.get("backend") != ident:
                        raise ValueError("provider and availability identities disagree")
                if any(e.backend_id() == ident for e in self._entries):
                    raise ValueError(f"duplicate backend ID: {ident}")
                self._entries.append(entry)
                return self
            except BaseException:
                (entry if entry is not None else integration).close()
                raise

    def build(self) -> Engine:
        with self._lock:
            if self._state != "OPEN":
                raise RuntimeError("engine builder is spent or closed")
            if not self._entries:
                self._close_entries()
                self._state = "CLOSED"
                raise ValueError("at least one backend integration is required")
            engine = Engine(self._entries)
            self._entries = []
            self._state = "SPENT"
            return engine

    def _close_entries(self):
        for e in self._entries:
            e.close()
        self._entries = []

    def close(self) -> None:
        with self._lock:
            if self._state == "OPEN":
                self._state = "CLOSED"
                self._close_entries()
