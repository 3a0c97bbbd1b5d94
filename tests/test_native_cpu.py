"""CPU-side checks: the C-ABI library loads and exports every declared symbol, the program image
encoding matches the runtime's packed layout, and host-side validation mirrors the reference."""
import ctypes
import re
import struct
from pathlib import Path

import numpy as np
import pytest

from synaptik_amd import native
from synaptik_amd.program import ProgramBuilder, OP_GEMM, OP_OPTIMIZER, OP_STEP_COMMIT
from synaptik_amd.training import (Adam, AdamW, Dense, MlpSpec, Sgd, lower_forward,
                                   lower_training_step)

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "synaptik_hip.h").read_text()
    return sorted(set(re.findall(r"\b(shk_hip_[a-z_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(native.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = native.load_library()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.shk_hip_abi_version() == native.ABI_VERSION


def test_calls_without_device_report_status_not_crash():
    lib = native.load_library()
    # null out-pointers and foreign handles are rejected with INVALID_ARGUMENT
    assert lib.shk_hip_context_create(0, None) == 1
    assert lib.shk_hip_buffer_release(None) == 1
    bogus = ctypes.c_void_p(ctypes.addressof(ctypes.create_string_buffer(64)))
    assert lib.shk_hip_program_release(bogus) == 1
    buf = ctypes.create_string_buffer(256)
    assert lib.shk_hip_last_error(buf, 256) == 0


def test_status_mapping_follows_metal_classes():
    lib = native.load_library()
    with pytest.raises(native.HipInvalidArgument):
        native.check(lib, 1)
    with pytest.raises(native.HipAllocationError):
        native.check(lib, 4)
    with pytest.raises(native.HipArithmeticError):
        native.check(lib, 15)
    with pytest.raises(native.HipIndexError):
        native.check(lib, 16)
    with pytest.raises(native.HipBackendError):
        native.check(lib, 11)


def test_image_layout():
    pb = ProgramBuilder()
    a = pb.input(6)
    b = pb.input(6, inout=True)
    c = pb.output(4)
    t = pb.internal(2, "i64")
    pb.gemm(a, b, c, 2, 2, 3, trans_b=True)
    pb.optimizer(t, [(b, a, None, None, 6)], kind="sgd", phase=0, lr=0.5)
    img = pb.image()
    magic, version, n_slots, n_steps = struct.unpack_from("<IIII", img, 0)
    assert (magic, version, n_slots, n_steps) == (0x504B4853, 1, 4, 2)
    slots = [struct.unpack_from("<QIIII", img, 16 + 24 * i) for i in range(4)]
    assert slots[0] == (24, 1, 0, 0, 0) and slots[1] == (24, 3, 1, 0, 0)
    assert slots[2] == (16, 2, 0, 0, 0) and slots[3] == (16, 0, 0, 2, 0)
    off = 16 + 24 * 4
    step = struct.unpack_from("<II8i16q8f", img, off)
    assert step[0] == OP_GEMM and step[1] == 0 and list(step[2:7]) == [0, 1, 2, -1, -1]
    assert list(step[10:22]) == [2, 2, 3, 3, 3, 2, 2, 0, 1, 0, 0, 0]
    off += 200
    step2 = struct.unpack_from("<II8i16q8f", img, off)
    assert step2[0] == OP_OPTIMIZER and step2[1] == 40
    assert struct.unpack_from("<iiiiiiiiq", img, off + 200) == (1, 0, -1, -1, -1, -1, -1, 0, 6)
    assert len(img) == off + 200 + 40


def test_training_lowering_structure():
    spec = MlpSpec.chain([4096] * 6, hidden="relu")
    pb, lay = lower_training_step(spec, 4096, Sgd(0.01, momentum=0.9))
    ops = [s.opcode for s in pb.steps]
    assert ops.count(OP_GEMM) == 14  # 5 forward, 5 dW, 4 dX
    assert ops.count(OP_OPTIMIZER) == 1 and ops[-1] == OP_STEP_COMMIT
    assert spec.parameter_count() == 83_906_560
    # inputs: current 5 W, 5 b, 10 momentum slots; candidate set of the same 20; counter, x, y
    assert pb.n_inputs == 43 and pb.n_outputs == 1
    pb2, lay2 = lower_training_step(MlpSpec.chain([784, 1024, 1024, 10], "relu", "ce"), 1024,
                                    Adam(1e-3))
    assert pb2.n_inputs == 2 * (6 + 6 + 6) + 3 and lay2.y.dtype == "i64"
    fwd = lower_forward(spec, 8)
    assert [s.opcode for s in fwd.steps] == [OP_GEMM] * 5


def test_optimizer_configuration_validation_mirrors_reference():
    with pytest.raises(ValueError):
        Sgd(0.1, momentum=1.0)
    with pytest.raises(ValueError):
        Sgd(0.1, nesterov=True)
    with pytest.raises(ValueError):
        Sgd(0.1, momentum=0.5, dampening=0.1, nesterov=True)
    with pytest.raises(ValueError):
        Sgd(-1.0)
    with pytest.raises(ValueError):
        Adam(1e-3, beta1=1.0)
    assert AdamW(1e-3).decoupled and not Adam(1e-3).decoupled
    with pytest.raises(ValueError):
        MlpSpec([Dense(3, 4), Dense(5, 2)])
    with pytest.raises(ValueError):
        Dense(3, 4, "gelu")


def test_library_exports_the_host_initialization_symbols():
    text = (ROOT / "include" / "synaptik_init.h").read_text()
    names = sorted(set(re.findall(r"\b(shk_lxm_[a-z_0-9]+)\s*\(", text)))
    assert names == ["shk_lxm_gaussian_tables", "shk_lxm_next_double", "shk_lxm_next_gaussian",
                     "shk_lxm_next_long", "shk_lxm_seed", "shk_lxm_uniform_f32",
                     "shk_lxm_uniform_f64"]
    lib = native.load_library()
    for name in names:
        assert hasattr(lib, name), name


def test_image_validation_without_a_device():
    """shk_hip_program_validate decodes an image as program creation does; it reports one run's
    arena size, rejects hostile extents, and survives degenerate steps."""
    from synaptik_amd.native import HipInvalidArgument, validate_program_image
    pb = ProgramBuilder()
    x, o = pb.input(5 * 4), pb.output(4)
    t = pb.internal(1000)
    pb.colsum(x, o, 5, 4)
    pb.copy(x, t, 20)
    arena = validate_program_image(pb.image())
    assert arena >= 256 + 1000 * 4 and arena % 256 == 0
    # a zero-width column sum once divided by zero while sizing its scratch
    pb = ProgramBuilder()
    x, o = pb.input(4), pb.output(1)
    pb.colsum(x, o, 5, 0, ldx=1)
    validate_program_image(pb.image())
    # extents whose products overflow int64 must be refused, not wrap into a passing bound
    for R, C, ld in ((2**40, 4, 2**30), (3, 2**62, 2**62)):
        pb = ProgramBuilder()
        x, o = pb.input(16), pb.output(16)
        pb.colsum(x, o, R, C, ldx=ld)
        with pytest.raises(HipInvalidArgument):
            validate_program_image(pb.image())
    pb = ProgramBuilder()
    x, y = pb.input(16), pb.output(16)
    pb.row_reduce(x, y, 2**31 - 1, 2**40, "sum")
    with pytest.raises(HipInvalidArgument):
        validate_program_image(pb.image())


def test_classifier_head_step_validation_without_a_device():
    """The fused classifier head step: a well-formed head validates; more than 16 classes, an
    unknown activation or phase, a written slot used twice, a read-only output and short slots
    are refused at decode time."""
    from synaptik_amd.native import HipBackendError, validate_program_image

    def head(R=8, K=12, J=4, act="relu", reuse=False, short=False, phase=None, ro=False):
        pb = ProgramBuilder()
        H, W, b = pb.input(R * K), pb.input(J * K - (1 if short else 0)), pb.input(J)
        t = pb.input(R, "i64")
        dz = pb.input(R * J) if ro else pb.internal(R * J)
        dx = dz if reuse else pb.internal(R * K)
        rl, loss = pb.internal(R), pb.output(1)
        st = pb.ce_head(H, W, t, dz, rl, R, K, J, bias=b, dx=dx, act=act)
        if phase is not None:
            st.iargs[4] = phase
        pb.ce_head_loss(rl, loss, R)
        return pb.image()

    assert validate_program_image(head()) > 0
    assert validate_program_image(head(J=16, K=9)) > 0
    for bad in (dict(J=17), dict(J=0), dict(reuse=True), dict(short=True), dict(phase=2),
                dict(ro=True)):
        with pytest.raises(HipBackendError):
            validate_program_image(head(**bad))
    pb = ProgramBuilder()
    rl = pb.internal(8)
    pb.ce_head_loss(rl, rl, 8)  # the loss may not alias its input
    with pytest.raises(HipBackendError):
        validate_program_image(pb.image())
