"""ctypes binding of libsynaptik_hip.so: the host-side mirror of the reference's FFM binding.

Mirrors `MetalNativeApi.Ffm` (modules/backend/metal/src/main/java/io/github/pho001/synaptik/
backend/metal/MetalNativeApi.java:3582-3700): the library is looked up once, its ABI version is
checked, every call returns an int32 status, and non-OK statuses become exceptions with the
same meaning as the Metal mapping (MetalNativeApi.java:482-507): invalid argument / range ->
IllegalArgument-like ValueError, allocation -> MemoryError, arithmetic -> ArithmeticError, the
rest -> HipBackendError.

There is deliberately no CPU fallback: if the library is missing, loading fails loudly.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import numpy as np

LIBRARY_PATH = Path(__file__).resolve().parent / "libsynaptik_hip.so"
ABI_VERSION = 1

STATUS_NAMES = {
    0: "OK",
    1: "INVALID_ARGUMENT",
    2: "NO_DEVICE",
    3: "NO_COMMAND_QUEUE",
    4: "ALLOCATION_FAILED",
    5: "RANGE_OUT_OF_BOUNDS",
    6: "COPY_FAILED",
    7: "INTERNAL_ERROR",
    8: "UNSUPPORTED_SHAPE",
    9: "GRAPH_COMPILATION_FAILED",
    10: "INCOMPATIBLE_RESOURCE",
    11: "EXECUTION_FAILED",
    12: "KERNEL_COMPILATION_FAILED",
    13: "UNSUPPORTED_OPERATION",
    14: "DEVICE_ERROR",
    15: "ARITHMETIC",
    16: "INDEX_OUT_OF_BOUNDS",
}

EXPORTED_SYMBOLS = (
    "shk_hip_abi_version",
    "shk_hip_last_error",
    "shk_hip_context_create",
    "shk_hip_context_release",
    "shk_hip_device_info",
    "shk_hip_buffer_create",
    "shk_hip_buffer_wrap",
    "shk_hip_buffer_release",
    "shk_hip_buffer_upload",
    "shk_hip_buffer_download",
    "shk_hip_buffer_device_pointer",
    "shk_hip_buffer_upload_staged",
    "shk_hip_buffer_download_canonical",
    "shk_hip_storage_transfer_bytes",
    "shk_hip_buffer_upload_storage",
    "shk_hip_buffer_download_storage",
    "shk_hip_program_create",
    "shk_hip_program_release",
    "shk_hip_program_run",
    "shk_hip_program_run_async",
    "shk_hip_program_wait",
    "shk_hip_program_set_concurrent",
    "shk_hip_program_side_steps",
    "shk_hip_program_arena_bytes",
    "shk_hip_program_lease_count",
    "shk_hip_program_run_static",
    "shk_hip_program_validate",
    "shk_hip_program_plan",
    "shk_hip_program_set_profiling",
    "shk_hip_program_step_times",
    "shk_hip_program_step_count",
    "shk_hip_program_set_graph_mode",
    "shk_hip_program_graph_mode",
)


class HipBackendError(RuntimeError):
    """A native status other than the argument, allocation and arithmetic classes."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class HipInvalidArgument(HipBackendError, ValueError):
    pass


class HipAllocationError(HipBackendError, MemoryError):
    pass


class HipArithmeticError(HipBackendError, ArithmeticError):
    pass


class HipIndexError(HipBackendError, ValueError):
    """Index target out of bounds (Java: IllegalArgumentException)."""


_lib = None
_lib_lock = threading.Lock()


def load_library(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Loads the library once and checks its ABI version. Raises if it is absent."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path is not None else LIBRARY_PATH
        if not p.exists():
            raise FileNotFoundError(
                f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        lib = ctypes.CDLL(str(p))
        vp = ctypes.c_void_p
        u64 = ctypes.c_uint64
        i32 = ctypes.c_int32
        u32 = ctypes.c_uint32
        sig = {
            "shk_hip_abi_version": (u32, []),
            "shk_hip_last_error": (i32, [ctypes.c_char_p, u64]),
            "shk_hip_context_create": (i32, [i32, ctypes.POINTER(vp)]),
            "shk_hip_context_release": (i32, [vp]),
            "shk_hip_device_info": (i32, [vp, ctypes.POINTER(i32), ctypes.POINTER(i32),
                                          ctypes.POINTER(u64), ctypes.c_char_p, u64]),
            "shk_hip_buffer_create": (i32, [vp, u64, ctypes.POINTER(vp)]),
            "shk_hip_buffer_wrap": (i32, [vp, vp, u64, ctypes.POINTER(vp)]),
            "shk_hip_buffer_release": (i32, [vp]),
            "shk_hip_buffer_upload": (i32, [vp, u64, vp, u64]),
            "shk_hip_buffer_download": (i32, [vp, u64, vp, u64]),
            "shk_hip_buffer_device_pointer": (i32, [vp, ctypes.POINTER(vp)]),
            "shk_hip_buffer_upload_staged": (i32, [vp, u64, vp, u64]),
            "shk_hip_buffer_download_canonical": (i32, [vp, u32, i32, u32,
                                                        ctypes.POINTER(ctypes.c_int64),
                                                        ctypes.POINTER(ctypes.c_int64),
                                                        ctypes.c_int64, vp, u64, u64]),
            "shk_hip_storage_transfer_bytes": (i32, [u32, u32, ctypes.POINTER(ctypes.c_int64),
                                                     ctypes.POINTER(ctypes.c_int64),
                                                     ctypes.c_int64, ctypes.POINTER(u64)]),
            "shk_hip_buffer_upload_storage": (i32, [vp, u32, i32, u32,
                                                    ctypes.POINTER(ctypes.c_int64),
                                                    ctypes.POINTER(ctypes.c_int64),
                                                    ctypes.c_int64, vp, u64]),
            "shk_hip_buffer_download_storage": (i32, [vp, u32, i32, u32,
                                                      ctypes.POINTER(ctypes.c_int64),
                                                      ctypes.POINTER(ctypes.c_int64),
                                                      ctypes.c_int64, vp, u64]),
            "shk_hip_program_create": (i32, [vp, vp, u64, ctypes.POINTER(vp)]),
            "shk_hip_program_release": (i32, [vp]),
            "shk_hip_program_run": (i32, [vp, u32, ctypes.POINTER(vp), u32, ctypes.POINTER(vp)]),
            "shk_hip_program_run_async": (i32, [vp, u32, ctypes.POINTER(vp), u32, ctypes.POINTER(vp)]),
            "shk_hip_program_wait": (i32, [vp]),
            "shk_hip_program_set_concurrent": (i32, [vp, i32]),
            "shk_hip_program_side_steps": (i32, [vp, ctypes.POINTER(u32)]),
            "shk_hip_program_arena_bytes": (i32, [vp, ctypes.POINTER(u64)]),
            "shk_hip_program_lease_count": (i32, [vp, ctypes.POINTER(u32)]),
            "shk_hip_program_validate": (i32, [vp, u64, ctypes.POINTER(u64)]),
            "shk_hip_program_plan": (i32, [vp, u64, u32, ctypes.POINTER(ctypes.c_uint8),
                                           ctypes.POINTER(ctypes.c_int32),
                                           ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(u32)]),
            "shk_hip_program_run_static": (i32, [vp, u32, ctypes.POINTER(vp), u32,
                                                 ctypes.POINTER(vp)]),
            "shk_hip_program_set_profiling": (i32, [vp, i32]),
            "shk_hip_program_step_times": (i32, [vp, ctypes.POINTER(ctypes.c_double), u32,
                                                 ctypes.POINTER(u64)]),
            "shk_hip_program_step_count": (i32, [vp, ctypes.POINTER(u32)]),
            "shk_hip_program_set_graph_mode": (i32, [vp, i32]),
            "shk_hip_program_graph_mode": (i32, [vp, ctypes.POINTER(i32)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.shk_hip_abi_version()
        if version != ABI_VERSION:
            raise HipBackendError(7, f"ABI version {version} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def _last_error(lib) -> str:
    buf = ctypes.create_string_buffer(512)
    lib.shk_hip_last_error(buf, 512)
    return buf.value.decode(errors="replace")


def check(lib, status: int) -> None:
    """Maps a native status to the exception class the Java binding would throw."""
    if status == 0:
        return
    msg = _last_error(lib)
    if status in (1, 5, 8, 10):
        raise HipInvalidArgument(status, msg)
    if status == 4:
        raise HipAllocationError(status, msg)
    if status == 15:
        raise HipArithmeticError(status, msg)
    if status == 16:
        raise HipIndexError(status, msg)
    raise HipBackendError(status, msg)


class HipContext:
    """One device and one stream (`shk_hip_context_create`)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = ctypes.c_void_p()
        check(self.lib, self.lib.shk_hip_context_create(device, ctypes.byref(h)))
        self.handle = h
        self.device = device

    def device_info(self) -> dict:
        cu = ctypes.c_int32()
        clk = ctypes.c_int32()
        mem = ctypes.c_uint64()
        name = ctypes.create_string_buffer(128)
        check(self.lib, self.lib.shk_hip_device_info(self.handle, ctypes.byref(cu), ctypes.byref(clk),
                                                     ctypes.byref(mem), name, 128))
        return {"compute_units": cu.value, "clock_khz": clk.value, "memory_bytes": mem.value,
                "arch": name.value.decode()}

    def buffer(self, nbytes: int) -> "HipBuffer":
        return HipBuffer(self, nbytes)

    def upload(self, array: np.ndarray) -> "HipBuffer":
        a = np.ascontiguousarray(array)
        b = HipBuffer(self, a.nbytes)
        b.upload(a)
        return b

    def close(self) -> None:
        if self.handle:
            check(self.lib, self.lib.shk_hip_context_release(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _geometry(shape, strides):
    shape = tuple(int(d) for d in shape)
    rank = len(shape)
    dims = (ctypes.c_int64 * max(1, rank))(*shape)
    st = None if strides is None else (ctypes.c_int64 * max(1, rank))(*[int(x) for x in strides])
    return dims, st, rank


def validate_program_image(image: bytes) -> int:
    """Decodes and validates a program image without a device (`shk_hip_program_validate`);
    returns the per-run arena bytes of one lease, or raises the status program creation would."""
    lib = load_library()
    out = ctypes.c_uint64()
    buf = ctypes.create_string_buffer(bytes(image), max(1, len(image)))
    check(lib, lib.shk_hip_program_validate(buf, len(image), ctypes.byref(out)))
    return out.value


def program_plan(image: bytes):
    """The two-stream schedule program creation gives an image, without a device
    (`shk_hip_program_plan`): (stream per step, the step each waits for or -1, the steps folded
    into the run's last launch: [loss MEAN or -1, optimizer pass or -1])."""
    lib = load_library()
    buf = ctypes.create_string_buffer(bytes(image), max(1, len(image)))
    n = ctypes.c_uint32()
    folded = (ctypes.c_int64 * 2)()
    st = lib.shk_hip_program_plan(buf, len(image), 0, None, None, folded, ctypes.byref(n))
    if n.value == 0:
        check(lib, st)
        return [], [], [-1, -1]
    streams = (ctypes.c_uint8 * n.value)()
    waits = (ctypes.c_int32 * n.value)()
    check(lib, lib.shk_hip_program_plan(buf, len(image), n.value, streams, waits, folded,
                                        ctypes.byref(n)))
    return list(streams), list(waits), list(folded)


def storage_transfer_bytes(element_width: int, shape, strides, storage_offset: int) -> int:
    """Byte extent of a storage-layout transfer of this geometry, 0 when it is not one
    (`shk_hip_storage_transfer_bytes`, host-only). Extents or offsets outside int64 are not
    representable and give 0."""
    lim = 1 << 63
    vals = [int(d) for d in shape] + [int(x) for x in (strides or ())] + [int(storage_offset)]
    if any(not -lim <= v < lim for v in vals) or len(tuple(shape)) > 16:
        return 0
    lib = load_library()
    dims, st, rank = _geometry(shape, strides)
    out = ctypes.c_uint64()
    check(lib, lib.shk_hip_storage_transfer_bytes(int(element_width), rank, dims, st,
                                                  int(storage_offset), ctypes.byref(out)))
    return out.value


class HipBuffer:
    """Device buffer handle (`shk_hip_buffer_*`); released exactly once."""

    def __init__(self, ctx: HipContext, nbytes: int, wrap_pointer: int | None = None):
        self.ctx = ctx
        self.lib = ctx.lib
        self.nbytes = int(nbytes)
        h = ctypes.c_void_p()
        if wrap_pointer is None:
            check(self.lib, self.lib.shk_hip_buffer_create(ctx.handle, self.nbytes, ctypes.byref(h)))
        else:
            check(self.lib, self.lib.shk_hip_buffer_wrap(ctx.handle, ctypes.c_void_p(wrap_pointer),
                                                         self.nbytes, ctypes.byref(h)))
        self.handle = h

    def upload(self, array: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(array)
        check(self.lib, self.lib.shk_hip_buffer_upload(self.handle, offset, a.ctypes.data, a.nbytes))

    def upload_staged(self, array: np.ndarray, offset: int = 0) -> None:
        """Upload through the context's pinned staging ring on its copy stream
        (`shk_hip_buffer_upload_staged`): returns once `array` has been read; the DMA may still be
        in flight and every later use of this buffer waits for it."""
        a = np.ascontiguousarray(array)
        check(self.lib, self.lib.shk_hip_buffer_upload_staged(self.handle, offset, a.ctypes.data, a.nbytes))

    def download(self, dtype=np.float32, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        check(self.lib, self.lib.shk_hip_buffer_download(self.handle, offset, out.ctypes.data, out.nbytes))
        return out

    def download_canonical(self, element_width: int, shape, strides=None, storage_offset: int = 0,
                           boolean: bool = False, maximum_bytes: int | None = None) -> memoryview:
        """Dense row-major big-endian bytes of a (possibly strided) view of this buffer
        (`shk_hip_buffer_download_canonical`), as a fresh read-only buffer (the reference hands
        out a read-only ByteBuffer over its private copy, HostTensorValue.bytes())."""
        shape = tuple(int(d) for d in shape)
        rank = len(shape)
        count = 0 if any(d == 0 for d in shape) else int(np.prod(shape, dtype=np.int64)) if shape else 1
        nbytes = count * (1 if boolean else int(element_width))
        if maximum_bytes is None:
            maximum_bytes = nbytes
        dims = (ctypes.c_int64 * max(1, rank))(*shape)
        st = None if strides is None else (ctypes.c_int64 * max(1, rank))(*[int(x) for x in strides])
        out = np.empty(max(1, nbytes), np.uint8)
        check(self.lib, self.lib.shk_hip_buffer_download_canonical(
            self.handle, int(element_width), 1 if boolean else 0, rank, dims, st,
            int(storage_offset), out.ctypes.data, nbytes, int(maximum_bytes)))
        return memoryview(out[:nbytes]).toreadonly()

    def upload_storage(self, element_width: int, shape, strides, storage_offset: int,
                       source, boolean: bool = False) -> None:
        """Writes the whole physical span of a storage-layout view from host bytes
        (`shk_hip_buffer_upload_storage`); BOOL logical elements are validated first."""
        src = np.ascontiguousarray(source).reshape(-1).view(np.uint8)
        dims, st, rank = _geometry(shape, strides)
        check(self.lib, self.lib.shk_hip_buffer_upload_storage(
            self.handle, int(element_width), 1 if boolean else 0, rank, dims, st,
            int(storage_offset), src.ctypes.data if src.nbytes else None, src.nbytes))

    def download_storage(self, element_width: int, shape, strides, storage_offset: int,
                         destination: np.ndarray, boolean: bool = False) -> None:
        """Reads the whole physical span of a storage-layout view into `destination`, a writable
        C-contiguous host array (`shk_hip_buffer_download_storage`); a BOOL view is validated on
        the device before any byte is written."""
        if not (destination.flags.c_contiguous and destination.flags.writeable):
            raise ValueError("destination must be writable contiguous host storage")
        dims, st, rank = _geometry(shape, strides)
        check(self.lib, self.lib.shk_hip_buffer_download_storage(
            self.handle, int(element_width), 1 if boolean else 0, rank, dims, st,
            int(storage_offset), destination.ctypes.data if destination.nbytes else None,
            destination.nbytes))

    def device_pointer(self) -> int:
        p = ctypes.c_void_p()
        check(self.lib, self.lib.shk_hip_buffer_device_pointer(self.handle, ctypes.byref(p)))
        return p.value or 0

    def close(self) -> None:
        if self.handle:
            check(self.lib, self.lib.shk_hip_buffer_release(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipBinding:
    """Prepared handle arrays of a program run's inputs and outputs (HipProgram.bind)."""
    __slots__ = ("ins", "outs", "n_in", "n_out", "buffers")

    def __init__(self, inputs, outputs):
        self.buffers = (tuple(inputs), tuple(outputs))
        self.n_in, self.n_out = len(inputs), len(outputs)
        self.ins = (ctypes.c_void_p * max(1, self.n_in))(*[b.handle.value for b in inputs])
        self.outs = (ctypes.c_void_p * max(1, self.n_out))(*[b.handle.value for b in outputs])


class HipProgram:
    """A created program (`shk_hip_program_create`) bound to a context."""

    def __init__(self, ctx: HipContext, image: bytes):
        self.ctx = ctx
        self.lib = ctx.lib
        buf = ctypes.create_string_buffer(image, len(image))
        h = ctypes.c_void_p()
        check(self.lib, self.lib.shk_hip_program_create(ctx.handle, buf, len(image), ctypes.byref(h)))
        self.handle = h

    def run(self, inputs, outputs) -> None:
        ins = (ctypes.c_void_p * max(1, len(inputs)))(*[b.handle.value for b in inputs])
        outs = (ctypes.c_void_p * max(1, len(outputs)))(*[b.handle.value for b in outputs])
        check(self.lib, self.lib.shk_hip_program_run(self.handle, len(inputs), ins, len(outputs), outs))

    def bind(self, inputs, outputs) -> "HipBinding":
        """The handle arrays of one set of bindings, built once for repeated runs
        (`run_bound`); the binding keeps its buffers referenced. The native call validates the
        bindings on every run as `run` does."""
        return HipBinding(inputs, outputs)

    def run_bound(self, binding: "HipBinding") -> None:
        check(self.lib, self.lib.shk_hip_program_run(self.handle, binding.n_in, binding.ins,
                                                     binding.n_out, binding.outs))

    def run_static(self, inputs, outputs) -> None:
        """One run whose per-run device memory is the library's static per-device array
        (`shk_hip_program_run_static`): allocates nothing; programs needing more than its
        64 MiB are refused."""
        ins = (ctypes.c_void_p * max(1, len(inputs)))(*[b.handle.value for b in inputs])
        outs = (ctypes.c_void_p * max(1, len(outputs)))(*[b.handle.value for b in outputs])
        check(self.lib, self.lib.shk_hip_program_run_static(self.handle, len(inputs), ins,
                                                            len(outputs), outs))

    def run_async(self, inputs, outputs) -> None:
        """Enqueues one run and returns (`shk_hip_program_run_async`); `wait` completes it."""
        ins = (ctypes.c_void_p * max(1, len(inputs)))(*[b.handle.value for b in inputs])
        outs = (ctypes.c_void_p * max(1, len(outputs)))(*[b.handle.value for b in outputs])
        check(self.lib, self.lib.shk_hip_program_run_async(self.handle, len(inputs), ins, len(outputs), outs))

    def set_concurrent(self, enabled: bool) -> None:
        """Two-stream step schedule on (the default) or off (`shk_hip_program_set_concurrent`)."""
        check(self.lib, self.lib.shk_hip_program_set_concurrent(self.handle, 1 if enabled else 0))

    def side_steps(self) -> int:
        """Steps the active schedule runs on the context's second stream."""
        v = ctypes.c_uint32()
        check(self.lib, self.lib.shk_hip_program_side_steps(self.handle, ctypes.byref(v)))
        return v.value

    def wait(self) -> None:
        """Completes the pending asynchronous run, raising its failure (`shk_hip_program_wait`)."""
        check(self.lib, self.lib.shk_hip_program_wait(self.handle))

    def lease_count(self) -> int:
        """Per-run leases (arena, status word, events, graphs) the program has created."""
        v = ctypes.c_uint32()
        check(self.lib, self.lib.shk_hip_program_lease_count(self.handle, ctypes.byref(v)))
        return v.value

    def arena_bytes(self) -> int:
        v = ctypes.c_uint64()
        check(self.lib, self.lib.shk_hip_program_arena_bytes(self.handle, ctypes.byref(v)))
        return v.value

    def step_count(self) -> int:
        v = ctypes.c_uint32()
        check(self.lib, self.lib.shk_hip_program_step_count(self.handle, ctypes.byref(v)))
        return v.value

    def set_graph_mode(self, enabled: bool) -> None:
        check(self.lib, self.lib.shk_hip_program_set_graph_mode(self.handle, 1 if enabled else 0))

    def graph_mode(self) -> bool:
        v = ctypes.c_int32(0)
        check(self.lib, self.lib.shk_hip_program_graph_mode(self.handle, ctypes.byref(v)))
        return v.value != 0

    def set_profiling(self, enabled: bool) -> None:
        check(self.lib, self.lib.shk_hip_program_set_profiling(self.handle, 1 if enabled else 0))

    def step_times(self):
        n = self.step_count()
        arr = (ctypes.c_double * max(1, n))()
        runs = ctypes.c_uint64()
        check(self.lib, self.lib.shk_hip_program_step_times(self.handle, arr, n, ctypes.byref(runs)))
        return list(arr)[:n], runs.value

    def close(self) -> None:
        if self.handle:
            check(self.lib, self.lib.shk_hip_program_release(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
