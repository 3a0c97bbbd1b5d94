"""Host-side mirror of the reference's backend SPI for the HIP backend.

The reference's Java SPI (modules/planning, modules/prepare, modules/runtime) is:
  * BackendCapabilityProvider.supports(OperationCapabilityQuery)
        (modules/planning/.../capability/BackendCapabilityProvider.java:19-56) - pure, per node;
  * BackendPartitionPreparer.analyze(PrepareContext) -> BackendPartitionAnalysis(plan, requirements)
        (modules/prepare/.../analysis/BackendPartitionPreparer.java:19-34);
  * BackendPartitionFinalizer.finalizePartition(...) -> (PreparedExecutable, PreparedResource[])
        (modules/prepare/.../BackendPartitionFinalizer.java:20-45), rolling back its own
        acquisitions on failure;
  * PreparedExecutable.bind(RunState) -> BoundInvocation, BoundInvocation.execute() synchronous
        (modules/runtime/.../execution/PreparedExecutable.java:254-313, BoundInvocation.java:51-68).
This module provides the same roles with the same names, over a small node-list IR standing in
for the compiler's PrepareContext (one planned partition: values with descriptors, nodes in
topological order, caller inputs and published outputs).

Lowering (what HipPartitionPreparer.analyze does):
  * MATMUL with a rank-2 PERMUTE operand absorbs the permute as a transpose flag;
  * PERMUTE(MATMUL(a, b)) is emitted as the swapped GEMM b^T-a^T writing the permuted result
    directly (the dW = PERMUTE(X^T . dZ) pattern of LinearAlgebraGradientRules.java:97-104);
  * MATMUL -> ADD(row bias) -> RELU/TANH/SIGMOID with single consumers becomes one GEMM with its
    epilogue (TensorLinearExpressions.java:97-146 builds exactly this chain);
  * maximal single-consumer elementwise chains of one shape become one POINTWISE step (<= 6 inputs,
    <= 2 outputs, <= 8 registers, <= 48 instructions), broadcast operands loaded in place;
  * SUM / MEAN / MAX / LOG_SUM_EXP over the last axis -> ROW_REDUCE, over all -> REDUCE_ALL,
    SUM_TO_SHAPE / SUM over rows -> COLSUM, SOFTMAX / LOG_SOFTMAX -> SOFTMAX,
    MEAN_SQUARED_ERROR -> MSE, INDEX_CATEGORICAL_CROSS_ENTROPY_WITH_LOGITS -> CE_INDEX;
  * any other PERMUTE [1,0] is materialized by the tiled transpose kernel.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from .native import (HipBuffer, HipContext, HipProgram, storage_transfer_bytes,
                     validate_program_image)
from .program import ProgramBuilder, Slot

BACKEND_ID = "hip"
DEVICE_CLASS = "ACCELERATOR"

ELEMENTWISE_UNARY = {"NEG": "neg", "RELU": "relu", "TANH": "tanh", "SIGMOID": "sigmoid",
                     "EXP": "exp", "LOG": "log", "SQRT": "sqrt"}
ELEMENTWISE_BINARY = {"ADD": "add", "SUB": "sub", "MUL": "mul", "DIV": "div", "MAXIMUM": "max",
                      "GREATER_THAN": "gt"}
ACTIVATIONS = {"RELU": "relu", "TANH": "tanh", "SIGMOID": "sigmoid"}
DTYPE_SLOT = {"FLOAT32": "f32", "INT32": "i32", "INT64": "i64", "BOOL": "f32"}
# Storage widths of the publishable types (DataType.byteWidth); FP8 is rejected like Metal does
# (MetalBackendRuntime.requireStorageType).
STORAGE_WIDTH = {"FLOAT64": 8, "FLOAT32": 4, "BFLOAT16": 2, "FLOAT16": 2, "INT64": 8, "INT32": 4,
                 "BOOL": 1}
UNSUPPORTED_STORAGE = ("FLOAT8_E4M3", "FLOAT8_E5M2")


class UnsupportedPartition(ValueError):
    """The partition holds a node this backend cannot lower (UNSUPPORTED_OPERATION)."""


@dataclass(frozen=True)
class TensorDescriptor:
    """Logical type and shape; `strides` / `storage_offset` (element units) describe a view's
    storage layout (None: dense row-major), as LayoutDescriptor does in the reference."""
    dtype: str
    shape: tuple
    strides: Optional[tuple] = None
    storage_offset: int = 0
    # False: the layout is not resolved yet (Optional.empty() in TensorDescriptor.layout())
    layout_resolved: bool = True

    @property
    def count(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1


@dataclass(frozen=True)
class OperationCapabilityQuery:
    """One compiled node as planning asks about it (OperationCapabilityQuery.java:50-253)."""
    kind: str
    inputs: tuple
    outputs: tuple
    attrs: tuple = ()

    def attr(self, name, default=None):
        return dict(self.attrs).get(name, default)


@dataclass
class Node:
    kind: str
    inputs: list
    output: str
    attrs: dict = field(default_factory=dict)


@dataclass
class Partition:
    """A planned single-owner partition: value descriptors, topologically ordered nodes, caller
    inputs (bound per run) and published outputs."""
    values: dict
    nodes: list
    inputs: list
    outputs: list


def _rank2(d: TensorDescriptor) -> bool:
    return len(d.shape) == 2


def _broadcastable(small: tuple, full: tuple) -> Optional[str]:
    """Broadcast mode of an operand of shape `small` against output `full`, or None."""
    if small == full:
        return "full"
    if small in ((), (1,), (1, 1)):
        return "scalar"
    if len(full) == 2:
        R, C = full
        if small in ((C,), (1, C)):
            return "row"
        if small == (R, 1):
            return "col"
    if len(full) == 1 and small == (1,):
        return "scalar"
    return None


class HipCapabilityProvider:
    """BackendCapabilityProvider for the HIP backend: pure and thread-safe."""

    def backend_id(self) -> str:
        return BACKEND_ID

    def supports(self, q: OperationCapabilityQuery) -> bool:
        ins, outs = q.inputs, q.outputs
        f32 = lambda d: d.dtype == "FLOAT32"  # noqa: E731
        if len(outs) != 1:
            return False
        out = outs[0]
        k = q.kind
        if k == "MATMUL":
            return (len(ins) == 2 and all(f32(d) and _rank2(d) for d in ins)
                    and ins[0].shape[1] == ins[1].shape[0] and f32(out))
        if k == "PERMUTE":
            return len(ins) == 1 and f32(ins[0]) and _rank2(ins[0]) and tuple(q.attr("axes", ())) == (1, 0)
        if k in ELEMENTWISE_UNARY:
            return len(ins) == 1 and f32(ins[0]) and f32(out) and ins[0].shape == out.shape and len(out.shape) <= 2
        if k in ELEMENTWISE_BINARY:
            ok_out = f32(out) or (k == "GREATER_THAN" and out.dtype == "BOOL")
            return (len(ins) == 2 and all(f32(d) for d in ins) and ok_out and len(out.shape) <= 2
                    and all(_broadcastable(d.shape, out.shape) for d in ins))
        if k == "WHERE":
            return (len(ins) == 3 and ins[0].dtype in ("BOOL", "FLOAT32") and f32(ins[1]) and f32(ins[2])
                    and len(out.shape) <= 2 and all(_broadcastable(d.shape, out.shape) for d in ins))
        if k == "EXPAND":
            return len(ins) == 1 and f32(ins[0]) and _broadcastable(ins[0].shape, out.shape) is not None
        if k == "CONSTANT":
            return len(ins) == 0 and f32(out) and len(out.shape) <= 2
        if k in ("SUM", "MEAN", "MAX"):
            if len(ins) != 1 or not f32(ins[0]) or len(ins[0].shape) > 2:
                return False
            axes = q.attr("axes")
            last = ((len(ins[0].shape) - 1,), (-1,))
            if k == "MAX":
                return axes is None or tuple(axes) in last
            return axes is None or tuple(axes) in last + ((0,),)
        if k == "SUM_TO_SHAPE":
            return (len(ins) == 1 and f32(ins[0]) and _rank2(ins[0])
                    and out.shape in ((ins[0].shape[1],), (1, ins[0].shape[1])))
        if k in ("LOG_SUM_EXP", "SOFTMAX", "LOG_SOFTMAX"):
            return (len(ins) == 1 and f32(ins[0]) and _rank2(ins[0])
                    and q.attr("axis", -1) in (-1, 1))
        if k == "MEAN_SQUARED_ERROR":
            return (len(ins) == 2 and all(f32(d) for d in ins) and ins[0].shape == ins[1].shape
                    and q.attr("reduction", "MEAN") in ("MEAN", "SUM"))
        if k == "INDEX_CATEGORICAL_CROSS_ENTROPY_WITH_LOGITS":
            return (len(ins) == 2 and f32(ins[0]) and _rank2(ins[0])
                    and ins[1].dtype in ("INT32", "INT64") and ins[1].shape == (ins[0].shape[0],)
                    and q.attr("reduction", "MEAN") == "MEAN" and q.attr("axis", -1) in (-1, 1))
        return False


@dataclass
class PreparationResourceRequirement:
    """Buffer(value, size, align) / Workspace(id, size, align) (PreparationResourceRequirement.java:16-179)."""
    kind: str
    ident: str
    byte_size: int
    alignment: int = 256


@dataclass
class BackendPartitionAnalysis:
    partition: Partition
    plan: bytes
    requirements: list
    input_slots: list
    output_slots: list


class HipPartitionPreparer:
    """BackendPartitionPreparer: lowers one partition to a program image (no device work)."""

    def __init__(self, provider: Optional[HipCapabilityProvider] = None):
        self.provider = provider or HipCapabilityProvider()

    def analyze(self, context) -> BackendPartitionAnalysis:
        """context: a PrepareContext (engine.py) or directly its partition graph."""
        part = context.graph if hasattr(context, "graph") else context
        lw = _Lowering(part, self.provider)
        pb, ins, outs = lw.lower()
        image = pb.image()
        internal = validate_program_image(image)  # one run's lease arena, no device needed
        reqs = [PreparationResourceRequirement("Buffer", v, part.values[v].count * 4 if part.values[v].dtype != "INT64" else part.values[v].count * 8)
                for v in part.outputs]
        reqs.append(PreparationResourceRequirement("Workspace", "arena", internal))
        return BackendPartitionAnalysis(part, image, reqs, ins, outs)


class HipPartitionFinalizer:
    """BackendPartitionFinalizer: creates the device program; releases it if anything fails.
    With a trace producer set (HipBackendIntegration.set_trace_observer), every prepared
    executable gets a trace unit and every bound run emits its plan, timing and outcome."""

    def __init__(self, ctx: HipContext):
        self.ctx = ctx
        self.tracer = None

    def finalize_partition(self, analysis: BackendPartitionAnalysis) -> "HipPreparedExecutable":
        program = HipProgram(self.ctx, analysis.plan)
        try:
            unit = self.tracer.prepare_unit() if self.tracer is not None else None
            return HipPreparedExecutable(self.ctx, program, analysis, unit)
        except Exception:
            program.close()
            raise


class BoundInvocation:
    """One bound run: execute() is synchronous and returns the published output buffers."""

    def __init__(self, exe: "HipPreparedExecutable", inputs: list, outputs: list):
        self.exe, self.inputs, self.outputs = exe, inputs, outputs

    def execute(self) -> list:
        exe = self.exe
        if exe.trace_unit is None:
            exe.program.run(self.inputs, self.outputs)
        else:
            from .trace import TracedRun
            a = exe.analysis
            TracedRun(exe.trace_unit.producer, exe.trace_unit, len(self.inputs),
                      len(self.outputs), sum(1 for r in a.requirements if r.kind == "Workspace"),
                      sum(b.nbytes for b in self.inputs), sum(s.nbytes for s in a.output_slots),
                      sum(r.byte_size for r in a.requirements if r.kind == "Workspace"))(
                lambda: exe.program.run(self.inputs, self.outputs))
        return self.outputs


class HipPreparedExecutable:
    """PreparedExecutable: immutable, shared across runs; per-run outputs come from fresh buffers
    (the run's representations), the internal arena is owned by the program resource."""

    def __init__(self, ctx: HipContext, program: HipProgram, analysis: BackendPartitionAnalysis,
                 trace_unit=None):
        self.ctx = ctx
        self.program = program
        self.analysis = analysis
        self.part = analysis.partition
        self.trace_unit = trace_unit

    def bind(self, inputs: dict, outputs: Optional[list] = None) -> BoundInvocation:
        """inputs: value id -> HipBuffer (accepted representations are this context's buffers);
        outputs: the run's buffers for the published values in order (created per run by the
        schedule's buffer creators), or None to create them here."""
        bufs = []
        for v in self.part.inputs:
            b = inputs.get(v)
            if not isinstance(b, HipBuffer) or b.ctx is not self.ctx:
                raise ValueError(f"input {v} is not a buffer of this backend's context")
            if b.nbytes < self.part.values[v].count * (8 if self.part.values[v].dtype == "INT64" else 4):
                raise ValueError(f"input {v} buffer is too small")
            bufs.append(b)
        if outputs is None:
            outs = [self.ctx.buffer(max(s.nbytes, 4)) for s in self.analysis.output_slots]
        else:
            outs = list(outputs)
            if len(outs) != len(self.analysis.output_slots):
                raise ValueError("one buffer per published value is required")
            for b, s in zip(outs, self.analysis.output_slots):
                if not isinstance(b, HipBuffer) or b.ctx is not self.ctx or b.nbytes < s.nbytes:
                    raise ValueError("an output representation is not an adequate buffer of "
                                     "this backend's context")
        return BoundInvocation(self, bufs, outs)

    def run_values(self, values: dict) -> dict:
        """Engine.runValues analogue: borrow host arrays, run, publish host arrays."""
        bufs = {}
        for v in self.part.inputs:
            d = self.part.values[v]
            np_dt = {"FLOAT32": np.float32, "INT32": np.int32, "INT64": np.int64}[d.dtype]
            bufs[v] = self.ctx.upload(np.ascontiguousarray(values[v], np_dt).reshape(-1))
        outs = self.bind(bufs).execute()
        res = {}
        for v, b in zip(self.part.outputs, outs):
            d = self.part.values[v]
            res[v] = b.download(np.float32, d.count).reshape(d.shape)
        return res

    def close(self):
        self.program.close()


def storage_transfer_extent(descriptor: TensorDescriptor) -> int:
    """Physical byte extent of a storage-layout transfer of `descriptor`, 0 when it is not one:
    unresolved layout, FP8, or a geometry MetalBackendRuntime.isStorageTransfer
    (MetalBackendRuntime.java:429-478) rejects. Computed by the native library's host code."""
    if descriptor is None:
        raise TypeError("descriptor must not be None")
    if not descriptor.layout_resolved or descriptor.dtype not in STORAGE_WIDTH:
        return 0
    return storage_transfer_bytes(STORAGE_WIDTH[descriptor.dtype], descriptor.shape,
                                  descriptor.strides, descriptor.storage_offset)


class HipBackendIntegration:
    """HipBackendIntegration.open(config): context + SPI roles (MetalBackendIntegration.java:50-103)."""

    def __init__(self, device: int = 0):
        self.context = HipContext(device)
        self.capability_provider = HipCapabilityProvider()
        self.preparer = HipPartitionPreparer(self.capability_provider)
        self.finalizer = HipPartitionFinalizer(self.context)

    @classmethod
    def open(cls, device: int = 0) -> "HipBackendIntegration":
        return cls(device)

    def set_trace_observer(self, observer) -> None:
        """Routes invocation trace records (synaptik_amd/trace.py) of executables prepared from
        now on to observer(record); None stops tracing new preparations."""
        from .trace import HipTraceProducer
        self.finalizer.tracer = None if observer is None else HipTraceProducer(
            observer, BACKEND_ID, int(self.context.device))

    def availability_snapshot(self) -> dict:
        info = self.context.device_info()
        return {"backend": BACKEND_ID, "device_class": DEVICE_CLASS, "device": info}

    def prepare(self, part: Partition) -> HipPreparedExecutable:
        return self.finalizer.finalize_partition(self.preparer.analyze(part))

    def _require_open(self):
        if not self.context.handle:
            raise RuntimeError("HIP device context is closed")  # IllegalStateException

    @staticmethod
    def _require_storage_type(dtype: str) -> int:
        if dtype in UNSUPPORTED_STORAGE or dtype not in STORAGE_WIDTH:
            raise ValueError(f"HIP does not support storage type {dtype}")
        return STORAGE_WIDTH[dtype]

    def borrow(self, dtype: str, storage: np.ndarray) -> HipBuffer:
        """Uploads caller host storage into a new device buffer owned by the caller
        (MetalBackendRuntime.borrow, MetalBackendRuntime.java:173-200): raw storage bytes, BOOL
        not interpreted here; FP8 rejected before any allocation."""
        self._require_storage_type(dtype)
        self._require_open()
        raw = np.ascontiguousarray(storage).view(np.uint8).reshape(-1)
        buf = HipBuffer(self.context, raw.nbytes)
        try:
            if raw.nbytes:
                buf.upload(raw)
        except BaseException:
            buf.close()
            raise
        return buf

    def copy_to_canonical_host_bytes(self, buffer: HipBuffer, descriptor: TensorDescriptor,
                                     maximum_bytes: int) -> memoryview:
        """Canonical dense row-major big-endian bytes of a publication
        (MetalBackendRuntime.copyToCanonicalHostBytes, MetalBackendRuntime.java:304-424;
        HostTensorValue.java:18): raw bits kept, BOOL elements must be 0 or 1, strided views
        gathered in row-major order. Packing runs on the device."""
        if buffer is None or descriptor is None:
            raise TypeError("buffer and descriptor must not be None")  # NullPointerException
        width = self._require_storage_type(descriptor.dtype)
        self._require_open()
        if maximum_bytes < 0:
            raise ValueError("maximumBytes must be non-negative")
        if buffer.ctx is not self.context or not buffer.handle:
            raise ValueError("representation must be a live readable buffer owned by this HIP integration")
        return buffer.download_canonical(width, descriptor.shape, descriptor.strides,
                                         descriptor.storage_offset,
                                         boolean=descriptor.dtype == "BOOL",
                                         maximum_bytes=maximum_bytes)

    # ---- prepared storage-layout transfers (MetalBackendIntegration.java:200-265) ----
    def storage_transfer_extent(self, descriptor: TensorDescriptor) -> int:
        return storage_transfer_extent(descriptor)

    def accepts_storage_layout_transfer(self, buffer: HipBuffer,
                                        descriptor: TensorDescriptor) -> bool:
        """Whether `buffer` is a live buffer of this context whose byte size is exactly the
        transfer extent of `descriptor` (MetalBackendRuntime.acceptsStorageLayoutTransfer,
        MetalBackendRuntime.java:211-223)."""
        if buffer is None or descriptor is None:
            raise TypeError("representation and descriptor must not be None")
        extent = self.storage_transfer_extent(descriptor)
        return (extent > 0 and isinstance(buffer, HipBuffer) and buffer.ctx is self.context
                and bool(buffer.handle) and buffer.nbytes == extent)

    def _transfer_args(self, buffer, descriptor, what):
        if not self.accepts_storage_layout_transfer(buffer, descriptor):
            raise ValueError(f"HIP {what} requires an exact live storage representation")
        return (STORAGE_WIDTH[descriptor.dtype], descriptor.shape, descriptor.strides,
                descriptor.storage_offset, descriptor.dtype == "BOOL")

    def bind_storage_layout_upload(self, buffer: HipBuffer, descriptor: TensorDescriptor):
        """Cold-binds `buffer` as the destination of a physical storage-layout upload
        (MetalBackendRuntime.bindStorageLayoutUpload, MetalBackendRuntime.java:233-247). The
        returned action takes host storage of at least the extent; BOOL logical elements are
        validated before the device is written."""
        width, shape, strides, offset, boolean = self._transfer_args(buffer, descriptor, "upload")

        def upload(source: np.ndarray) -> None:
            buffer.upload_storage(width, shape, strides, offset, source, boolean=boolean)
        return upload

    def bind_storage_layout_download(self, buffer: HipBuffer, descriptor: TensorDescriptor):
        """Cold-binds `buffer` as the source of a physical storage-layout download
        (MetalBackendRuntime.bindStorageLayoutDownload, MetalBackendRuntime.java:260-281): the
        action writes the whole span into writable host storage; a BOOL view is validated on the
        device first and a non-canonical byte leaves the destination untouched."""
        width, shape, strides, offset, boolean = self._transfer_args(buffer, descriptor, "download")

        def download(destination: np.ndarray) -> None:
            buffer.download_storage(width, shape, strides, offset, destination, boolean=boolean)
        return download

    def close(self):
        self.context.close()


class BoundBufferTransfer:
    """One bound per-run transfer action (BoundBufferTransfer.java; the Bound class of
    CpuMetalPreparedBufferTransfer.java:222-249): retains the host storage and the device
    action, allocates nothing when executed."""

    def __init__(self, host: np.ndarray, action):
        self._host = host
        self._action = action

    def execute(self) -> None:
        self._action(self._host)


class CpuHipPreparedBufferTransfer:
    """Immutable CPU<->HIP storage-layout transfer recipe for one prepared logical value
    (CpuMetalPreparedBufferTransfer.java:16-250, with the HIP integration in Metal's place).

    Construction checks the descriptor's geometry and that the prepared memory slot holds exactly
    its byte extent; `bind` validates both concrete representations (host storage: C-contiguous,
    exact byte size, writable when it is the destination; device: HipBackendIntegration's
    storage-transfer acceptance) and returns the bound action."""

    CPU_TO_HIP = "CPU_TO_HIP"
    HIP_TO_CPU = "HIP_TO_CPU"

    def __init__(self, hip: HipBackendIntegration, slot_bytes: int,
                 descriptor: TensorDescriptor, direction: str):
        if hip is None or descriptor is None or direction is None:
            raise TypeError("hip, descriptor and direction must not be None")
        if direction not in (self.CPU_TO_HIP, self.HIP_TO_CPU):
            raise ValueError(f"unknown CPU/HIP transfer direction {direction}")
        extent = hip.storage_transfer_extent(descriptor)
        if extent <= 0:
            raise ValueError("CPU/HIP transfer requires rank-0..16 static non-overlapping "
                             "positive-stride storage geometry with a checked byte extent")
        if int(slot_bytes) != extent:
            raise ValueError("transfer descriptor byte extent does not match prepared memory slot")
        self.hip = hip
        self.descriptor = descriptor
        self.direction = direction
        self.byte_count = extent

    @staticmethod
    def supports(descriptor: TensorDescriptor) -> bool:
        """CpuMetalPreparedBufferTransfer.supports (CpuMetalPreparedBufferTransfer.java:73-77)."""
        return storage_transfer_extent(descriptor) > 0

    @classmethod
    def cpu_to_hip(cls, hip, slot_bytes, descriptor):
        return cls(hip, slot_bytes, descriptor, cls.CPU_TO_HIP)

    @classmethod
    def hip_to_cpu(cls, hip, slot_bytes, descriptor):
        return cls(hip, slot_bytes, descriptor, cls.HIP_TO_CPU)

    def _accepts_host(self, host, writable: bool) -> bool:
        return (isinstance(host, np.ndarray) and host.flags.c_contiguous
                and host.nbytes == self.byte_count and (host.flags.writeable or not writable))

    def accepts_source(self, representation) -> bool:
        if self.direction == self.CPU_TO_HIP:
            return self._accepts_host(representation, False)
        return self.hip.accepts_storage_layout_transfer(representation, self.descriptor)

    def accepts_destination(self, representation) -> bool:
        if self.direction == self.CPU_TO_HIP:
            return self.hip.accepts_storage_layout_transfer(representation, self.descriptor)
        return self._accepts_host(representation, True)

    def bind(self, source, destination) -> BoundBufferTransfer:
        if not self.accepts_source(source) or not self.accepts_destination(destination):
            raise ValueError("incompatible buffer representation for this CPU/HIP transfer")
        if self.direction == self.CPU_TO_HIP:
            return BoundBufferTransfer(
                source, self.hip.bind_storage_layout_upload(destination, self.descriptor))
        return BoundBufferTransfer(
            destination, self.hip.bind_storage_layout_download(source, self.descriptor))


# ---------------------------------------------------------------------------------------------
class _Lowering:
    def __init__(self, part: Partition, provider: HipCapabilityProvider):
        self.p = part
        self.provider = provider
        self.pb = ProgramBuilder()
        self.slot: dict[str, Slot] = {}
        self.producer: dict[str, Node] = {n.output: n for n in part.nodes}
        self.uses: dict[str, list] = {}
        for n in part.nodes:
            for v in n.inputs:
                self.uses.setdefault(v, []).append(n)
        for v in part.outputs:
            self.uses.setdefault(v, []).append(None)  # publication counts as a use
        self.done: set = set()
        # EXPAND outputs are views of their source (loaded with a broadcast mode)
        self.bcast: dict[str, str] = {n.output: n.inputs[0] for n in part.nodes if n.kind == "EXPAND"}
        # PERMUTE [1,0] handling, decided up front:
        #   absorbed: every consumer is a MATMUL and the source is a stored value -> transpose flag;
        #   swapped:  a MATMUL whose only consumer is a non-absorbed PERMUTE writes the permuted
        #             result directly as the swapped GEMM.
        self.absorbed: set = set()
        self.swapped: set = set()
        for n in part.nodes:
            if n.kind != "PERMUTE":
                continue
            users = self.uses.get(n.output, [])
            src = self.producer.get(n.inputs[0])
            src_swaps = (src is not None and src.kind == "MATMUL"
                         and self.single_use(n.inputs[0]) is n and n.inputs[0] not in part.outputs)
            if users and all(u is not None and u.kind == "MATMUL" for u in users) and not src_swaps:
                self.absorbed.add(n.output)
            elif src_swaps:
                self.swapped.add(src.output)

    def d(self, v) -> TensorDescriptor:
        return self.p.values[v]

    def single_use(self, v) -> Optional[Node]:
        u = self.uses.get(v, [])
        return u[0] if len(u) == 1 and u[0] is not None else None

    def storage(self, v) -> Slot:
        """The slot holding value v (creating an internal or output slot as needed)."""
        v = self.bcast.get(v, v)
        if v not in self.slot:
            d = self.d(v)
            self.slot[v] = self.pb.internal(d.count, DTYPE_SLOT[d.dtype])
        return self.slot[v]

    def lower(self):
        for n in self.p.nodes:
            q = OperationCapabilityQuery(n.kind, tuple(self.d(v) for v in n.inputs), (self.d(n.output),),
                                         tuple(sorted((k, tuple(v) if isinstance(v, list) else v)
                                                      for k, v in n.attrs.items())))
            if not self.provider.supports(q):
                raise UnsupportedPartition(f"node {n.kind} -> {n.output} is not admitted")
        for v in self.p.inputs:
            d = self.d(v)
            self.slot[v] = self.pb.input(d.count, DTYPE_SLOT[d.dtype])
        out_slots = []
        for v in self.p.outputs:
            if v in self.slot:
                raise UnsupportedPartition(f"output {v} is also a caller input")
            d = self.d(v)
            self.slot[v] = self.pb.output(d.count, DTYPE_SLOT[d.dtype])
            out_slots.append(self.slot[v])
        groups = self._elementwise_groups()
        order = {n.output: i for i, n in enumerate(self.p.nodes)}
        last_of = {v: max(g, key=lambda m: order[m.output]).output for v, g in groups.items()}
        for n in self.p.nodes:
            if n.output in self.done:
                continue
            k = n.kind
            if k == "EXPAND":
                self.done.add(n.output)
                if n.output in self.p.outputs:
                    raise UnsupportedPartition("a broadcast view cannot be published directly")
            elif k == "PERMUTE":
                self._permute(n)
            elif k == "MATMUL":
                self._matmul(n)
            elif k in ELEMENTWISE_UNARY or k in ELEMENTWISE_BINARY or k in ("WHERE", "CONSTANT"):
                # a fused chain is emitted at its last node, after every operand it reads
                if last_of[n.output] == n.output:
                    self._pointwise(groups[n.output])
            else:
                self._reduction(n)
        return self.pb, [self.slot[v] for v in self.p.inputs], out_slots

    # ---- matmul family ----
    def _operand(self, v):
        """(value holding the rank-2 operand, transposed?) absorbing a PERMUTE producer."""
        if v in self.absorbed:
            return self.producer[v].inputs[0], True
        return v, False

    def _permute(self, n: Node):
        if n.output in self.absorbed:
            self.done.add(n.output)
            return
        src = n.inputs[0]
        R, C = self.d(src).shape
        self.pb.transpose(self.storage(src), self.storage(n.output), R, C)
        self.done.add(n.output)

    def _matmul(self, n: Node):
        a, ta = self._operand(n.inputs[0])
        b, tb = self._operand(n.inputs[1])
        M, K = self.d(n.inputs[0]).shape
        N = self.d(n.inputs[1]).shape[1]
        user = self.single_use(n.output)
        # PERMUTE(MATMUL(a, b)) = MATMUL(b^T, a^T): swap operands, flip transposes
        if n.output in self.swapped:
            self.pb.gemm(self.storage(b), self.storage(a), self.storage(user.output), N, M, K,
                         trans_a=not tb, trans_b=not ta)
            self.done.update({n.output, user.output})
            return
        bias, act, final = None, None, n.output
        if user is not None and user.kind == "ADD" and n.output not in self.p.outputs:
            other = user.inputs[1] if user.inputs[0] == n.output else user.inputs[0]
            src = self.bcast.get(other, other)
            if _broadcastable(self.d(src).shape, (M, N)) == "row" and self.d(src).count == N:
                bias, final = src, user.output
        nxt = self.single_use(final)
        if nxt is not None and nxt.kind in ACTIVATIONS and final not in self.p.outputs:
            act, final = ACTIVATIONS[nxt.kind], nxt.output
        self.pb.gemm(self.storage(a), self.storage(b), self.storage(final), M, N, K,
                     trans_a=ta, trans_b=tb, bias=self.storage(bias) if bias else None, act=act)
        self.done.add(n.output)
        if bias:
            self.done.add(user.output)
        if act:
            self.done.add(final)

    # ---- elementwise ----
    def _elementwise_groups(self) -> dict:
        """Union single-consumer elementwise chains of one output shape (union-find)."""
        parent = {}

        def find(x):
            while parent[x] != x:
                parent[x] = parent[parent[x]]
                x = parent[x]
            return x

        ew = [n for n in self.p.nodes if n.kind in ELEMENTWISE_UNARY or n.kind in ELEMENTWISE_BINARY
              or n.kind in ("WHERE", "CONSTANT")]
        for n in ew:
            parent[n.output] = n.output
        for n in ew:
            for v in n.inputs:
                pn = self.producer.get(v)
                if (pn is not None and v in parent and self.single_use(v) is n
                        and v not in self.p.outputs and self.d(v).shape == self.d(n.output).shape):
                    parent[find(v)] = find(n.output)
        groups: dict[str, list] = {}
        for n in ew:
            groups.setdefault(find(n.output), []).append(n)
        return {n.output: groups[find(n.output)] for n in ew}

    def _pointwise(self, group: list):
        if all(n.output in self.done for n in group):
            return
        # a node fused into a GEMM epilogue may sit in a group: keep only the unlowered ones
        nodes = [n for n in group if n.output not in self.done]
        try:
            self._emit_pointwise(nodes)
        except _TooBig:
            for n in nodes:
                self._emit_pointwise([n])

    def _emit_pointwise(self, nodes: list):
        produced = {n.output for n in nodes}
        out_shape = self.d(nodes[-1].output).shape
        shape2 = out_shape if len(out_shape) == 2 else ((1, out_shape[0]) if out_shape else (1, 1))
        R, C = shape2
        # external inputs and group outputs
        ext, outs = [], []
        for n in nodes:
            for v in n.inputs:
                src = self.bcast.get(v, v)
                if v not in produced and src not in ext:
                    ext.append(src)
        for n in nodes:
            users = self.uses.get(n.output, [])
            if any(u is None or u.output not in produced for u in users):
                outs.append(n.output)
        for n in nodes:
            if self.d(n.output).shape != out_shape:
                raise _TooBig()
        if len(ext) > 6 or len(outs) > 2:
            raise _TooBig()
        modes = []
        for v in ext:
            m = _broadcastable(self.d(v).shape, out_shape) if self.d(v).shape != out_shape else "full"
            if len(out_shape) < 2 and self.d(v).shape == out_shape:
                m = "full"
            if m is None:
                raise _TooBig()
            modes.append(m)
        code = []
        reg: dict[str, int] = {}
        free = list(range(8))
        last_use: dict[str, int] = {}
        for i, n in enumerate(nodes):
            for v in n.inputs:
                last_use[self.bcast.get(v, v) if v not in produced else v] = i

        def get(v, i):
            key = v if v in produced else self.bcast.get(v, v)
            if key not in reg:
                if not free:
                    raise _TooBig()
                r = free.pop(0)
                reg[key] = r
                code.append(("load", r, ext.index(key), 0, 0, 0.0))
            return reg[key]

        for i, n in enumerate(nodes):
            ins = [get(v, i) for v in n.inputs]
            for v in n.inputs:  # free registers of values dead after this node
                key = v if v in produced else self.bcast.get(v, v)
                if last_use.get(key) == i and key not in outs and key in reg:
                    free.append(reg.pop(key))
            if not free:
                raise _TooBig()
            r = free.pop(0)
            k = n.kind
            if k == "CONSTANT":
                code.append(("const", r, 0, 0, 0, float(n.attrs["value"])))
            elif k in ELEMENTWISE_UNARY:
                code.append((ELEMENTWISE_UNARY[k], r, ins[0], 0, 0, 0.0))
            elif k in ELEMENTWISE_BINARY:
                code.append((ELEMENTWISE_BINARY[k], r, ins[0], ins[1], 0, 0.0))
            elif k == "WHERE":
                code.append(("where", r, ins[1], ins[2], ins[0], 0.0))
            reg[n.output] = r
            if n.output in outs:
                code.append(("store", outs.index(n.output), r, 0, 0, 0.0))
            if n.output not in last_use and n.output in reg and n.output not in outs:
                free.append(reg.pop(n.output))
        if len(code) > 48:
            raise _TooBig()
        self.pb.pointwise(R, C, [self.storage(v) for v in ext], [self.storage(v) for v in outs], code,
                          modes=modes)
        self.done.update(produced)

    # ---- reductions, normalization, losses ----
    def _reduction(self, n: Node):
        k = n.kind
        x = n.inputs[0]
        dx = self.d(x)
        out = self.storage(n.output)
        if k in ("SUM", "MEAN", "MAX"):
            axes = n.attrs.get("axes")
            kind = k.lower()
            if axes is None or len(dx.shape) < 2 and tuple(axes) in ((0,), (-1,)):
                self.pb.reduce_all(self.storage(x), out, dx.count, kind)
            elif tuple(axes) in ((1,), (-1,)):
                self.pb.row_reduce(self.storage(x), out, dx.shape[0], dx.shape[1], kind)
            elif tuple(axes) == (0,) and k in ("SUM", "MEAN"):
                self.pb.colsum(self.storage(x), out, dx.shape[0], dx.shape[1], mean=(k == "MEAN"))
            else:
                raise UnsupportedPartition(f"{k} over axes {axes}")
        elif k == "SUM_TO_SHAPE":
            self.pb.colsum(self.storage(x), out, dx.shape[0], dx.shape[1])
        elif k == "LOG_SUM_EXP":
            self.pb.row_reduce(self.storage(x), out, dx.shape[0], dx.shape[1], "lse")
        elif k in ("SOFTMAX", "LOG_SOFTMAX"):
            self.pb.softmax(self.storage(x), out, dx.shape[0], dx.shape[1], log=(k == "LOG_SOFTMAX"))
        elif k == "MEAN_SQUARED_ERROR":
            self.pb.mse(self.storage(x), self.storage(n.inputs[1]), out, dx.count,
                        reduction=n.attrs.get("reduction", "MEAN").lower())
        elif k == "INDEX_CATEGORICAL_CROSS_ENTROPY_WITH_LOGITS":
            ign = n.attrs.get("ignore_index")
            self.pb.index_ce(self.storage(x), self.storage(n.inputs[1]), out, dx.shape[0], dx.shape[1],
                             ignore_index=ign)
        else:
            raise UnsupportedPartition(f"no lowering for {k}")
        self.done.add(n.output)


class _TooBig(Exception):
    pass
