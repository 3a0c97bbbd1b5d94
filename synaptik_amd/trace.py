"""Invocation tracing of the HIP backend, shaped like the reference's trace payloads.

* `BackendInvocationOutcome` (modules/trace/.../payload/BackendInvocationOutcome.java): backend,
  device, prepared-unit and invocation ids, SUCCEEDED / FAILED, the route kind and the native
  status, with the reference's consistency rule (SUCCEEDED needs a SUCCESS native status,
  FAILED forbids one; TraceNativeStatus: code 0 if and only if SUCCESS).
* `HipInvocationPlan`, the analogue of the Metal producer's invocation plan record
  (MetalTraceProducer.invocationPlanned): slot counts and aggregate input / output / internal
  bytes of the run, plus the run's wall time on the calling thread.
* `HipTraceProducer` mirrors MetalTraceProducer's protocol: ids come from atomic counters, each
  record goes to an observer, and an observer that raises disables the producer (tracing never
  changes the outcome of a run).
"""
from __future__ import annotations

import itertools
import threading
import time
from dataclasses import dataclass
from enum import Enum
from typing import Callable, Optional

# native status code (synaptik_hip.h) -> TraceNativeStatusKind
_NATIVE_KIND = {0: "SUCCESS", 1: "INVALID_ARGUMENT", 2: "DEVICE_UNAVAILABLE",
                3: "COMMAND_QUEUE_UNAVAILABLE", 4: "ALLOCATION_FAILED", 5: "RANGE_OUT_OF_BOUNDS",
                6: "COPY_FAILED", 7: "INTERNAL_ERROR", 8: "UNSUPPORTED_SHAPE",
                9: "COMPILATION_FAILED", 10: "INCOMPATIBLE_RESOURCE", 11: "EXECUTION_FAILED",
                12: "COMPILATION_FAILED", 14: "EXECUTION_FAILED"}
# 13 (UNSUPPORTED_OPERATION), 15 (ARITHMETIC) and 16 (INDEX_OUT_OF_BOUNDS) have no kind of their
# own in the reference's vocabulary: UNKNOWN, with the native code kept


class TraceOutcomeStatus(Enum):
    SUCCEEDED = "SUCCEEDED"
    FAILED = "FAILED"


class TraceRouteKind(Enum):
    CUSTOM_KERNEL = "CUSTOM_KERNEL"
    GRAPH_EXECUTABLE = "GRAPH_EXECUTABLE"


TRACE_NATIVE_STATUS_KINDS = ("SUCCESS", "INVALID_ARGUMENT", "DEVICE_UNAVAILABLE",
                             "COMMAND_QUEUE_UNAVAILABLE", "ALLOCATION_FAILED",
                             "RANGE_OUT_OF_BOUNDS", "COPY_FAILED", "INTERNAL_ERROR",
                             "UNSUPPORTED_SHAPE", "COMPILATION_FAILED", "INCOMPATIBLE_RESOURCE",
                             "EXECUTION_FAILED", "UNKNOWN")


@dataclass(frozen=True)
class TraceNativeStatus:
    kind: str
    code: int

    def __post_init__(self):
        if self.kind not in TRACE_NATIVE_STATUS_KINDS:
            raise ValueError(f"unknown native status kind {self.kind}")
        if self.kind == "SUCCESS" and self.code != 0:
            raise ValueError("SUCCESS requires code 0")
        if self.kind != "SUCCESS" and self.code == 0:
            raise ValueError("code 0 requires SUCCESS")

    @staticmethod
    def of(code: int) -> "TraceNativeStatus":
        return TraceNativeStatus(_NATIVE_KIND.get(int(code), "UNKNOWN"), int(code))


@dataclass(frozen=True)
class BackendInvocationOutcome:
    backend_id: str
    device_id: int
    prepared_unit_id: int
    invocation_id: int
    status: TraceOutcomeStatus
    route: TraceRouteKind
    native_status: Optional[TraceNativeStatus]

    def __post_init__(self):
        ok = self.native_status is not None and self.native_status.kind == "SUCCESS"
        if self.status is TraceOutcomeStatus.SUCCEEDED and not ok:
            raise ValueError("SUCCEEDED requires SUCCESS nativeStatus")
        if self.status is TraceOutcomeStatus.FAILED and ok:
            raise ValueError("FAILED forbids SUCCESS nativeStatus")


@dataclass(frozen=True)
class HipInvocationPlan:
    prepared_unit_id: int
    invocation_id: int
    route: TraceRouteKind
    feed_slot_count: int
    target_slot_count: int
    internal_slot_count: int
    aggregate_input_bytes: int
    aggregate_output_bytes: int
    aggregate_internal_bytes: int


@dataclass(frozen=True)
class HipInvocationTiming:
    """Wall time of one synchronous run on the calling thread (HIP addition)."""
    prepared_unit_id: int
    invocation_id: int
    wall_ms: float


@dataclass(frozen=True)
class PreparedUnit:
    producer: "HipTraceProducer"
    prepared_unit_id: int
    route: TraceRouteKind


class HipTraceProducer:
    """Emits trace records to `observer(record)`; disabled for good when the observer raises."""

    def __init__(self, observer: Callable, backend_id: str = "hip", device_id: int = 0):
        if observer is None:
            raise TypeError("observer")
        self._observer = observer
        self.backend_id, self.device_id = backend_id, device_id
        self._enabled = True
        self._lock = threading.Lock()
        self._units = itertools.count()
        self._invocations = itertools.count()

    @property
    def enabled(self) -> bool:
        return self._enabled

    def _emit(self, record) -> None:
        if not self._enabled:
            return
        try:
            self._observer(record)
        except Exception:  # noqa: BLE001 - tracing must not change the run
            self._enabled = False

    def prepare_unit(self, route: TraceRouteKind = TraceRouteKind.GRAPH_EXECUTABLE):
        if not self._enabled:
            return None
        with self._lock:
            return PreparedUnit(self, next(self._units), route)

    def begin_invocation(self, unit: PreparedUnit) -> Optional[int]:
        if not self._enabled or unit is None:
            return None
        if unit.producer is not self:
            raise ValueError("prepared trace unit belongs to another producer")
        with self._lock:
            return next(self._invocations)

    def invocation_planned(self, unit, invocation_id, feeds, targets, internals, in_bytes,
                           out_bytes, internal_bytes) -> None:
        if invocation_id is None:
            return
        self._emit(HipInvocationPlan(unit.prepared_unit_id, invocation_id, unit.route, feeds,
                                     targets, internals, in_bytes, out_bytes, internal_bytes))

    def invocation_completed(self, unit, invocation_id, native_code: int, wall_ms: float) -> None:
        if invocation_id is None:
            return
        self._emit(HipInvocationTiming(unit.prepared_unit_id, invocation_id, wall_ms))
        native = TraceNativeStatus.of(native_code)
        status = (TraceOutcomeStatus.SUCCEEDED if native.kind == "SUCCESS"
                  else TraceOutcomeStatus.FAILED)
        self._emit(BackendInvocationOutcome(self.backend_id, self.device_id,
                                            unit.prepared_unit_id, invocation_id, status,
                                            unit.route, native))


class TracedRun:
    """Brackets one synchronous native run with its plan, timing and outcome records."""

    def __init__(self, producer: Optional[HipTraceProducer], unit, feeds, targets, internals,
                 in_bytes, out_bytes, internal_bytes):
        self.producer, self.unit = producer, unit
        self.args = (feeds, targets, internals, in_bytes, out_bytes, internal_bytes)

    def __call__(self, run: Callable[[], None]) -> None:
        p = self.producer
        inv = p.begin_invocation(self.unit) if p is not None and p.enabled else None
        if inv is not None:
            p.invocation_planned(self.unit, inv, *self.args)
        t0 = time.perf_counter()
        code = 0
        try:
            run()
        except Exception as e:  # native failures carry their status; others are internal
            code = getattr(e, "status", 7) or 7
            raise
        finally:
            if inv is not None:
                p.invocation_completed(self.unit, inv, code, (time.perf_counter() - t0) * 1e3)
