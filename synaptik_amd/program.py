"""Program images: the op-list format `shk_hip_program_create` decodes.

This is the HIP analogue of the Metal backend's graph image (schema 22, decoded by
synaptik_metal_mpsgraph_executable_create, synaptik_metal_foundation.m:8573): a prepared
partition is lowered once to a flat list of kernel steps over numbered slots.

Layout (little-endian, packed):
    header  : u32 magic 'SHKP', u32 version=1, u32 n_slots, u32 n_steps
    slot[i] : u64 bytes, u32 kind, u32 ext_index, u32 dtype, u32 flags          (24 bytes)
    step[j] : u32 opcode, u32 payload_bytes, i32 slot[8], i64 iarg[16], f32 farg[8] (200 bytes)
              followed by payload_bytes of payload, zero-padded to a multiple of 8
Slot kinds: INTERNAL (program arena, zeroed once at create), INPUT (in[ext_index], read only),
OUTPUT (out[ext_index]), INOUT (in[ext_index], updated in place: parameters, optimizer slots and
the completed-step counter of a device-resident training program).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = 0x504B4853
VERSION = 1

INTERNAL, INPUT, OUTPUT, INOUT = 0, 1, 2, 3
DTYPES = {"f32": (0, 4), "i32": (1, 4), "i64": (2, 8), "u8": (3, 1), "f64": (4, 8)}
NP_DTYPES = {"f32": np.float32, "i32": np.int32, "i64": np.int64, "u8": np.uint8, "f64": np.float64}

OP_GEMM = 1
OP_COLSUM = 2
OP_ROW_REDUCE = 3
OP_REDUCE_ALL = 4
OP_POINTWISE = 5
OP_SOFTMAX = 6
OP_SOFTMAX_BWD = 7
OP_LSE_BWD = 8
OP_MSE = 9
OP_CE_INDEX = 10
OP_OPTIMIZER = 11
OP_STEP_COMMIT = 12
OP_FILL = 13
OP_COPY = 14
OP_TRANSPOSE = 15
OP_CE_HEAD = 16

ACT = {None: 0, "none": 0, "relu": 1, "tanh": 2, "sigmoid": 3}
REDUCE_KIND = {"sum": 0, "mean": 1, "max": 2, "lse": 3}

# pointwise register-machine opcodes (elementwise.hip)
PW = {
    "load": 0, "const": 1, "add": 2, "sub": 3, "mul": 4, "div": 5, "neg": 6,
    "relu": 7, "tanh": 8, "sigmoid": 9, "exp": 10, "log": 11,
    "relu_grad": 12, "tanh_grad": 13, "sigmoid_grad": 14, "gt": 15, "where": 16,
    "store": 17, "max": 18, "sqrt": 19,
}
BROADCAST = {"full": 0, "row": 1, "col": 2, "scalar": 3}

_STEP = struct.Struct("<II8i16q8f")
_SLOT = struct.Struct("<QIIII")
assert _STEP.size == 200 and _SLOT.size == 24


@dataclass
class Slot:
    index: int
    kind: int
    ext_index: int
    dtype: str
    count: int

    @property
    def nbytes(self) -> int:
        return self.count * DTYPES[self.dtype][1]


@dataclass
class Step:
    opcode: int
    slots: list = field(default_factory=lambda: [-1] * 8)
    iargs: list = field(default_factory=lambda: [0] * 16)
    fargs: list = field(default_factory=lambda: [0.0] * 8)
    payload: bytes = b""


def _sid(s) -> int:
    return -1 if s is None else (s.index if isinstance(s, Slot) else int(s))


class ProgramBuilder:
    """Builds a program image step by step; slots are created with input/output/internal."""

    def __init__(self):
        self.slots: list[Slot] = []
        self.steps: list[Step] = []
        self.n_inputs = 0
        self.n_outputs = 0

    # ---- slots ----
    def _slot(self, kind, count, dtype, ext) -> Slot:
        if dtype not in DTYPES:
            raise ValueError(f"unknown dtype {dtype}")
        s = Slot(len(self.slots), kind, ext, dtype, int(count))
        self.slots.append(s)
        return s

    def input(self, count: int, dtype: str = "f32", inout: bool = False) -> Slot:
        s = self._slot(INOUT if inout else INPUT, count, dtype, self.n_inputs)
        self.n_inputs += 1
        return s

    def output(self, count: int, dtype: str = "f32") -> Slot:
        s = self._slot(OUTPUT, count, dtype, self.n_outputs)
        self.n_outputs += 1
        return s

    def internal(self, count: int, dtype: str = "f32") -> Slot:
        return self._slot(INTERNAL, count, dtype, 0)

    def _add(self, opcode, slots=(), iargs=(), fargs=(), payload=b"") -> Step:
        st = Step(opcode)
        for i, s in enumerate(slots):
            st.slots[i] = _sid(s)
        for i, v in enumerate(iargs):
            st.iargs[i] = int(v)
        for i, v in enumerate(fargs):
            st.fargs[i] = float(v)
        st.payload = payload
        self.steps.append(st)
        return st

    # ---- steps ----
    def gemm(self, A, B, C, M, N, K, *, trans_a=False, trans_b=False, lda=None, ldb=None,
             ldc=None, bias=None, act=None, aux=None, act_grad=False, ldaux=None,
             accumulate=False, colsum=None, dy=None, dz=None) -> Step:
        """C = op(A).op(B) (+bias, act) or C = act_grad(act, op(A).op(B), aux); `colsum`
        optionally receives the column sums of the stored C (a bias gradient).

        With `dy` and `dz` (a forward GEMM with its cotangent), C = act(op(A).op(B) + bias) and
        dz = act_grad(act, dy, C) (dy and dz with leading dimension ldaux); `colsum` then
        receives the column sums of dz."""
        lda = lda if lda is not None else (M if trans_a else K)
        ldb = ldb if ldb is not None else (K if trans_b else N)
        ldc = ldc if ldc is not None else N
        ldaux = ldaux if ldaux is not None else N
        if (dy is None) != (dz is None):
            raise ValueError("dy and dz go together")
        if dy is not None and (act_grad or aux is not None or accumulate):
            raise ValueError("a forward GEMM with its cotangent has no aux, act_grad or accumulate")
        mode = 2 if dy is not None else (1 if act_grad else 0)
        return self._add(OP_GEMM, [A, B, C, bias, dy if dy is not None else aux, colsum, None, dz],
                         [M, N, K, lda, ldb, ldc, ldaux, int(trans_a), int(trans_b), ACT[act],
                          mode, 1 if accumulate else 0])

    def gemm_update(self, A, B, M, N, K, counter, tensor, *, kind: str, trans_a=False,
                    trans_b=False, lda=None, ldb=None, lr: float, momentum=0.0, dampening=0.0,
                    weight_decay=0.0, nesterov=False, has_momentum_slot=False, beta1=0.9,
                    beta2=0.999, eps=1e-8) -> Step:
        """G = op(A).op(B) consumed by a staged optimizer update in the GEMM epilogue.

        tensor = (param, m, v, param_next, m_next, v_next) over the row-major [M, N] result; the
        candidates are written exactly as OPTIMIZER phase 2 would from G, which is not stored."""
        k = {"sgd": 0, "adam": 1, "adamw": 2}[kind]
        lda = lda if lda is not None else (M if trans_a else K)
        ldb = ldb if ldb is not None else (K if trans_b else N)
        p, m, v, pn, mn, vn = tensor
        payload = struct.pack("<iiiiiiiiq", _sid(p), -1, _sid(m), _sid(v), _sid(pn), _sid(mn),
                              _sid(vn), 0, int(M) * int(N))
        return self._add(OP_GEMM, [A, B, None, None, None, None, counter],
                         [M, N, K, lda, ldb, N, N, int(trans_a), int(trans_b), 0, 0, 0, k,
                          int(nesterov), int(has_momentum_slot)],
                         [lr, momentum, dampening, weight_decay, beta1, beta2, eps], payload)

    def colsum(self, X, out, R, N, *, ldx=None, mean=False, accumulate=False) -> Step:
        return self._add(OP_COLSUM, [X, out], [R, N, ldx if ldx is not None else N,
                                               int(accumulate), int(mean)])

    def row_reduce(self, X, out, R, C, kind: str) -> Step:
        return self._add(OP_ROW_REDUCE, [X, out], [R, C, REDUCE_KIND[kind]])

    def reduce_all(self, X, out, n, kind: str) -> Step:
        return self._add(OP_REDUCE_ALL, [X, out], [n, REDUCE_KIND[kind]])

    def pointwise(self, R, C, inputs, outputs, code, modes=None) -> Step:
        """code: list of (op, dst, a, b, c, imm) tuples; inputs bind load sources 0..5."""
        if len(inputs) > 6 or len(outputs) > 2:
            raise ValueError("pointwise supports 6 inputs and 2 outputs")
        modes = list(modes or ["full"] * len(inputs))
        slots = list(inputs) + [None] * (6 - len(inputs)) + list(outputs) + [None] * (2 - len(outputs))
        iargs = [R, C] + [BROADCAST[m] for m in modes] + [0] * (6 - len(modes))
        payload = b"".join(
            struct.pack("<BBBBBBBBf", PW[op], dst, a, b, c, 0, 0, 0, imm)
            for (op, dst, a, b, c, imm) in code)
        return self._add(OP_POINTWISE, slots, iargs, payload=payload)

    def softmax(self, X, Y, R, C, *, lse=None, log=False) -> Step:
        return self._add(OP_SOFTMAX, [X, Y, lse], [R, C, int(log)])

    def softmax_bwd(self, Y, G, dX, R, C, *, rowscale=None, rowscale_const=0.0) -> Step:
        return self._add(OP_SOFTMAX_BWD, [Y, G, dX, rowscale], [R, C], [rowscale_const])

    def lse_bwd(self, X, lse, dX, R, C, *, g=None, gconst=1.0) -> Step:
        return self._add(OP_LSE_BWD, [X, lse, g, dX], [R, C], [gconst])

    def mse(self, P, T, loss, n, *, grad=None, g=1.0, reduction="mean") -> Step:
        return self._add(OP_MSE, [P, T, loss, grad], [n, {"mean": 0, "sum": 1}[reduction]], [g])

    def index_ce(self, logits, target, loss, R, C, *, grad=None, ignore_index=None, g=1.0) -> Step:
        is64 = 1 if (isinstance(target, Slot) and target.dtype == "i64") else 0
        return self._add(OP_CE_INDEX, [logits, target, loss, grad],
                         [R, C, is64, 0 if ignore_index is None else 1,
                          0 if ignore_index is None else ignore_index], [g])

    def ce_head(self, H, W, target, dz, row_loss, R, K, J, *, bias=None, logits=None, dx=None,
                act=None, g=1.0) -> Step:
        """Classifier head of a training step: logits = H . W^T + bias ([R, J], stored when
        `logits` is given), per-row index cross-entropy into `row_loss`, the logit cotangent
        dz = (softmax - onehot) * (g / R) and, when `dx` is given, the input cotangent
        act_grad(act, dz . W, H). J <= 16; MEAN without an ignore index."""
        is64 = 1 if (isinstance(target, Slot) and target.dtype == "i64") else 0
        return self._add(OP_CE_HEAD, [H, W, bias, target, logits, dz, dx, row_loss],
                         [R, K, J, ACT[act], 0, is64], [g])

    def ce_head_loss(self, row_loss, loss, R) -> Step:
        """MEAN of the head's per-row losses into loss[0]."""
        return self._add(OP_CE_HEAD, [row_loss, loss], [R, 0, 0, 0, 1])

    def optimizer(self, counter, tensors, *, kind: str, phase: int, lr: float, momentum=0.0,
                  dampening=0.0, weight_decay=0.0, nesterov=False, has_momentum_slot=False,
                  beta1=0.9, beta2=0.999, eps=1e-8) -> Step:
        """tensors: list of (param, grad, m, v, count) or, for phase 2 (staged into the other
        half of a double buffer), (param, grad, m, v, param_next, m_next, v_next, count) slots;
        absent slots are None. At most 16 tensors per step."""
        k = {"sgd": 0, "adam": 1, "adamw": 2, "acc_sum": 3, "acc_commit": 4, "acc_clear": 5}[kind]
        if len(tensors) > 16:
            raise ValueError("at most 16 tensors per optimizer step")
        rows = []
        for t in tensors:
            if len(t) == 5:
                p, g, m, v, n = t
                pn = mn = vn = None
            else:
                p, g, m, v, pn, mn, vn, n = t
            rows.append(struct.pack("<iiiiiiiiq", _sid(p), _sid(g), _sid(m), _sid(v), _sid(pn),
                                    _sid(mn), _sid(vn), 0, int(n)))
        payload = b"".join(rows)
        return self._add(OP_OPTIMIZER, [counter], [k, phase, int(nesterov), int(has_momentum_slot)],
                         [lr, momentum, dampening, weight_decay, beta1, beta2, eps], payload)

    def step_commit(self, counter) -> Step:
        return self._add(OP_STEP_COMMIT, [counter])

    def fill(self, X, n, value=0.0) -> Step:
        return self._add(OP_FILL, [X], [n], [value])

    def copy(self, src, dst, n) -> Step:
        return self._add(OP_COPY, [src, dst], [n])

    def transpose(self, X, Y, R, C) -> Step:
        """Y[C,R] = X[R,C]^T."""
        return self._add(OP_TRANSPOSE, [X, Y], [R, C])

    # ---- encoding ----
    def image(self) -> bytes:
        out = [struct.pack("<IIII", MAGIC, VERSION, len(self.slots), len(self.steps))]
        for s in self.slots:
            out.append(_SLOT.pack(s.nbytes, s.kind, s.ext_index, DTYPES[s.dtype][0], 0))
        for st in self.steps:
            out.append(_STEP.pack(st.opcode, len(st.payload), *st.slots, *st.iargs, *st.fargs))
            pad = (-len(st.payload)) % 8
            out.append(st.payload + b"\0" * pad)
        return b"".join(out)
