"""Device-resident training for fully-connected networks on the HIP backend.

Mirrors the reference's training surface for the MLP path:
  * optimizer configurations `Sgd`, `Adam`, `AdamW` with the reference's validation
    (modules/training/src/main/java/io/github/pho001/synaptik/training/Sgd.java:23-181,
     Adam.java:194-286);
  * `HipTrainingSession` ~ `TrainingSession` (TrainingSession.java:242-647): `open`, `run`
    (GradientMode.RESET_AND_STEP), `optimizer_steps`, `state()` / `restore()` with byte-exact
    parameter and optimizer slots (TrainingSession.java:680-760).

Unlike the reference, whose optimizer runs on the host after downloading every gradient
(TrainingSession.java:916-950, TrainingParameter.java:409-672), the whole step is ONE program:
forward GEMMs with fused bias+activation, the loss and its gradient, the backward GEMMs (dX with
the previous layer's activation gradient fused into the epilogue, dW written directly in [out,in]
order), the bias column sums, and the transactional fused optimizer update. Parameters, slots and
the completed-step counter stay in HBM; a run downloads only the objective.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from .native import HipBuffer, HipContext, HipProgram
from .program import ProgramBuilder, Slot

ACTIVATIONS = (None, "relu", "tanh", "sigmoid")

# Sum each hidden layer's bias gradient inside the epilogue of the dX GEMM that produces its
# cotangent (instead of a separate column-sum pass over it).
FUSE_BIAS_GRADIENT = True
# In RESET_AND_STEP runs, stage each weight's optimizer update in the epilogue of the GEMM that
# computes its gradient (the gradient is never stored and the weights skip the streaming pass).
FUSE_OPTIMIZER = True
# Lower a cross-entropy head of at most 16 classes to one fused step (logits, per-row loss, the
# logit cotangent and the cotangent of the head's input; bit-identical to the unfused steps).
FUSE_CE_HEAD = True


class GradientMode:
    """How one successful run uses its gradients (GradientMode.java):
    RESET_AND_STEP ignores and empties the pending accumulator and steps from this run;
    ACCUMULATE adds this run's gradients to the accumulator without stepping;
    ACCUMULATE_AND_STEP adds them, steps from the complete sum and empties the accumulator."""
    RESET_AND_STEP = "reset_and_step"
    ACCUMULATE = "accumulate"
    ACCUMULATE_AND_STEP = "accumulate_and_step"


# ---- optimizer configurations (immutable, validated like the reference records) ----
@dataclass(frozen=True)
class Sgd:
    """SGD with optional momentum, dampening, coupled weight decay and Nesterov (Sgd.java:23-181)."""
    learning_rate: float
    momentum: float = 0.0
    dampening: float = 0.0
    weight_decay: float = 0.0
    nesterov: bool = False

    def __post_init__(self):
        if not (math.isfinite(self.learning_rate) and self.learning_rate > 0):
            raise ValueError(f"learning rate must be finite and positive: {self.learning_rate}")
        if not (math.isfinite(self.momentum) and 0.0 <= self.momentum < 1.0):
            raise ValueError(f"momentum must be finite and in [0, 1): {self.momentum}")
        if not (math.isfinite(self.dampening) and 0.0 <= self.dampening <= 1.0):
            raise ValueError(f"dampening must be finite and in [0, 1]: {self.dampening}")
        if not (math.isfinite(self.weight_decay) and self.weight_decay >= 0.0):
            raise ValueError(f"weight decay must be finite and non-negative: {self.weight_decay}")
        if self.nesterov and (self.momentum <= 0.0 or self.dampening != 0.0):
            raise ValueError("Nesterov requires positive momentum and zero dampening")


@dataclass(frozen=True)
class Adam:
    """Adam with coupled L2 decay (Adam.java:194-286)."""
    learning_rate: float
    beta1: float = 0.9
    beta2: float = 0.999
    epsilon: float = 1e-8
    weight_decay: float = 0.0

    decoupled = False

    def __post_init__(self):
        if not (math.isfinite(self.learning_rate) and self.learning_rate > 0):
            raise ValueError("learning rate must be finite and positive")
        for name in ("beta1", "beta2"):
            v = getattr(self, name)
            if not (math.isfinite(v) and 0.0 <= v < 1.0):
                raise ValueError(f"{name} must be finite and in [0, 1): {v}")
        if not (math.isfinite(self.epsilon) and self.epsilon > 0):
            raise ValueError("epsilon must be finite and positive")
        if not (math.isfinite(self.weight_decay) and self.weight_decay >= 0):
            raise ValueError("weight decay must be finite and non-negative")


@dataclass(frozen=True)
class AdamW(Adam):
    """Adam with decoupled weight decay."""
    decoupled = True


# ---- model description ----
@dataclass
class Dense:
    """One Linear layer y = act(x . W^T + b) with W stored [out, in] (Linear.java:48-370)."""
    fan_in: int
    fan_out: int
    activation: str | None = None
    bias: bool = True

    def __post_init__(self):
        if self.activation not in ACTIVATIONS:
            raise ValueError(f"unsupported activation {self.activation}")
        if self.fan_in <= 0 or self.fan_out <= 0:
            raise ValueError("layer extents must be positive")


@dataclass
class MlpSpec:
    layers: list[Dense]
    loss: str = "mse"  # "mse" or "ce" (index categorical cross-entropy with logits)
    reduction: str = "mean"  # loss reduction: "mean" or "sum" (MSE only)

    def __post_init__(self):
        if not self.layers:
            raise ValueError("a network needs at least one layer")
        for a, b in zip(self.layers, self.layers[1:]):
            if a.fan_out != b.fan_in:
                raise ValueError("consecutive layer extents differ")
        if self.loss not in ("mse", "ce"):
            raise ValueError(f"unsupported loss {self.loss}")
        if self.reduction not in ("mean", "sum") or (self.loss == "ce" and self.reduction != "mean"):
            raise ValueError(f"unsupported reduction {self.reduction}")

    @staticmethod
    def chain(widths: Sequence[int], hidden: str | None, loss: str = "mse",
              output: str | None = None) -> "MlpSpec":
        layers = []
        for i, (a, b) in enumerate(zip(widths, widths[1:])):
            last = i == len(widths) - 2
            layers.append(Dense(a, b, output if last else hidden))
        return MlpSpec(layers, loss)

    def parameter_count(self) -> int:
        return sum(l.fan_in * l.fan_out + (l.fan_out if l.bias else 0) for l in self.layers)


def init_parameters(spec: MlpSpec, seed: int, scheme: str):
    """Seeded initial weights, biases zero.

    'builder': what `Model.builder().seed(seed)` creates for this Linear chain -- Glorot-uniform
    weights from one L64X128MixRandom per builder step (initializers.builder_parameters).
    'builder_he_normal': the same generators and step seeds with Linear's kaimingReluNormal policy
    (sigma sqrt(2 / fanIn), one nextGaussian per weight in row-major order).
    'xavier_uniform' (bound sqrt(6/(fan_in+fan_out))) and 'he_normal' (sigma sqrt(2/fan_in)) draw
    the same distributions as ParameterInitializers.java:269-372 from numpy's generator instead,
    for seeded synthetic inputs."""
    if scheme == "builder":
        from .initializers import builder_parameters
        return builder_parameters(spec, seed)
    if scheme == "builder_he_normal":
        from .initializers import ParameterInitialization, builder_parameters
        return builder_parameters(spec, seed, policy=ParameterInitialization("kaiming_relu_normal"))
    rng = np.random.default_rng(seed)
    Ws, bs = [], []
    for l in spec.layers:
        if scheme == "xavier_uniform":
            bound = math.sqrt(6.0 / (l.fan_in + l.fan_out))
            W = rng.uniform(-bound, bound, size=(l.fan_out, l.fan_in))
        elif scheme == "he_normal":
            W = rng.standard_normal((l.fan_out, l.fan_in)) * math.sqrt(2.0 / l.fan_in)
        else:
            raise ValueError(f"unknown init scheme {scheme}")
        Ws.append(W.astype(np.float32))
        bs.append(np.zeros(l.fan_out, np.float32) if l.bias else None)
    return Ws, bs


# ---- lowering ----
@dataclass
class TrainingLayout:
    """Slot handles of a lowered training program, in input-index order."""
    weights: list[Slot] = field(default_factory=list)
    biases: list[Slot] = field(default_factory=list)
    first: list[Slot] = field(default_factory=list)    # momentum / first-moment slots
    second: list[Slot] = field(default_factory=list)   # second-moment slots (Adam)
    # staged (double-buffered) update: candidate parameter and slot buffers the step writes
    weights_next: list[Slot] = field(default_factory=list)
    biases_next: list[Slot] = field(default_factory=list)
    first_next: list[Slot] = field(default_factory=list)
    second_next: list[Slot] = field(default_factory=list)
    accum: list[Slot] = field(default_factory=list)    # gradient accumulators (accumulating modes)
    counter: Slot | None = None
    x: Slot | None = None
    y: Slot | None = None
    loss: Slot | None = None
    grads: list[Slot] = field(default_factory=list)


def _optimizer_kind(opt) -> str:
    if isinstance(opt, Sgd):
        return "sgd"
    if isinstance(opt, Adam):
        return "adamw" if opt.decoupled else "adam"
    raise TypeError(f"unsupported optimizer {opt!r}")


def lower_training_step(spec: MlpSpec, batch: int, optimizer, *, label_dtype: str = "i64",
                        mode: str = GradientMode.RESET_AND_STEP, clear_accumulator: bool = False):
    """Lowers one training step of `spec` at `batch` rows to a program image.

    Inputs (in order): W_1..W_L, b_1..b_L (current, read only), first-moment slots per tensor
    (SGD with momentum and Adam), second-moment slots (Adam); for modes that step, the same
    tensors again as the candidate set the update writes (INOUT); gradient accumulators (INOUT,
    accumulating modes and RESET_AND_STEP with clear_accumulator), completed-step counter (INOUT,
    int64), x [batch, in], y ([batch, out] f32 for MSE; [batch] int for CE).
    Output: objective [1].

    The update reads the current set and writes the candidate set: for RESET_AND_STEP each
    weight's update runs in the epilogue of its gradient GEMM (FUSE_OPTIMIZER), the rest is one
    streaming pass after the backward sweep. The caller adopts the candidate set only when the run succeeds. Every mode is transactional: a
    non-finite accumulated candidate or optimizer intermediate leaves the current parameters,
    slots, accumulators and the counter unchanged.
    """
    kind = _optimizer_kind(optimizer)
    pb = ProgramBuilder()
    lay = TrainingLayout()
    L = len(spec.layers)
    steps = mode != GradientMode.ACCUMULATE
    for l in spec.layers:
        lay.weights.append(pb.input(l.fan_in * l.fan_out))
    for l in spec.layers:
        lay.biases.append(pb.input(l.fan_out) if l.bias else None)
    params = lay.weights + [b for b in lay.biases if b is not None]
    has_first = kind != "sgd" or optimizer.momentum != 0.0
    if has_first:
        lay.first = [pb.input(p.count) for p in params]
    if kind != "sgd":
        lay.second = [pb.input(p.count) for p in params]
    if steps:
        lay.weights_next = [pb.input(w.count, inout=True) for w in lay.weights]
        lay.biases_next = [pb.input(b.count, inout=True) if b is not None else None for b in lay.biases]
        if has_first:
            lay.first_next = [pb.input(p.count, inout=True) for p in params]
        if kind != "sgd":
            lay.second_next = [pb.input(p.count, inout=True) for p in params]
    uses_acc = mode != GradientMode.RESET_AND_STEP or clear_accumulator
    if uses_acc:
        lay.accum = [pb.input(p.count, inout=True) for p in params]
    lay.counter = pb.input(1, "i64", inout=True)
    lay.x = pb.input(batch * spec.layers[0].fan_in)
    out_w = spec.layers[-1].fan_out
    if spec.loss == "mse":
        lay.y = pb.input(batch * out_w)
    else:
        lay.y = pb.input(batch, label_dtype)
    lay.loss = pb.output(1)

    # activations Y_l (internal); Y_0 is the input x
    acts = [lay.x] + [pb.internal(batch * l.fan_out) for l in spec.layers]
    # one cotangent buffer per layer: reusing a buffer two layers apart would make the input
    # gradient of a layer wait (write after read) for the weight gradient of the layer above it,
    # serializing the two streams' work
    dz = [pb.internal(batch * l.fan_out) for l in spec.layers]
    gW = [pb.internal(l.fan_in * l.fan_out) for l in spec.layers]
    gb = [pb.internal(l.fan_out) if l.bias else None for l in spec.layers]
    lay.grads = gW + [g for g in gb if g is not None]

    # A cross-entropy head of at most 16 classes is one fused step (logits, loss, both
    # cotangents); its forward GEMM is not emitted separately.
    head = FUSE_CE_HEAD and spec.loss == "ce" and out_w <= 16
    # forward
    for i, l in enumerate(spec.layers[: L - 1] if head else spec.layers):
        pb.gemm(acts[i], lay.weights[i], acts[i + 1], batch, l.fan_out, l.fan_in, trans_b=True,
                bias=lay.biases[i], act=l.activation)
    # objective and its cotangent (g = 1)
    if spec.layers[-1].activation is not None:
        raise ValueError("the loss heads are lowered for an identity output layer "
                         "(cross-entropy consumes raw logits)")
    dx_done = False  # the head also produced the cotangent of the last layer's input
    head_loss = None
    if spec.loss == "mse":
        pb.mse(acts[L], lay.y, lay.loss, batch * out_w, grad=dz[L - 1], reduction=spec.reduction)
    elif head:
        row_loss = pb.internal(batch)
        last = spec.layers[-1]
        pb.ce_head(acts[L - 1], lay.weights[L - 1], lay.y, dz[L - 1], row_loss, batch,
                   last.fan_in, out_w, bias=lay.biases[L - 1],
                   dx=dz[L - 2] if L > 1 else None,
                   act=spec.layers[L - 2].activation if L > 1 else None)
        head_loss = (row_loss, lay.loss, batch)
        dx_done = L > 1
    else:
        pb.index_ce(acts[L], lay.y, lay.loss, batch, out_w, grad=dz[L - 1])
    common = {}
    if kind == "sgd":
        common = dict(lr=optimizer.learning_rate, momentum=optimizer.momentum,
                      dampening=optimizer.dampening, weight_decay=optimizer.weight_decay,
                      nesterov=optimizer.nesterov, has_momentum_slot=has_first)
    else:
        common = dict(lr=optimizer.learning_rate, beta1=optimizer.beta1, beta2=optimizer.beta2,
                      eps=optimizer.epsilon, weight_decay=optimizer.weight_decay)
    fuse_update = FUSE_OPTIMIZER and mode == GradientMode.RESET_AND_STEP
    # backward. The two-stream plan keeps a step on the main stream when it depends on the main
    # stream's latest step, so the emission order shapes the schedule: first the chain of input
    # cotangents (each layer's waits on the one above), then every layer's weight and bias
    # gradients, which start as soon as their own cotangent exists and run beside the chain.
    db_fused = [False] * L  # db_i was summed in the epilogue of the GEMM producing dZ_i
    for i in reversed(range(1, L)):
        if dx_done and i == L - 1:
            continue
        l, prev = spec.layers[i], spec.layers[i - 1]
        # dZ_{i-1} = act_grad(dZ_i . W_i, Y_{i-1}), with db_{i-1} = SUM_TO_SHAPE(dZ_{i-1}) summed
        # in the same epilogue
        fuse = FUSE_BIAS_GRADIENT and gb[i - 1] is not None
        pb.gemm(dz[i], lay.weights[i], dz[i - 1], batch, l.fan_in, l.fan_out, aux=acts[i],
                act=prev.activation or "none", act_grad=True, colsum=gb[i - 1] if fuse else None)
        db_fused[i - 1] = fuse
    for i in reversed(range(L)):
        l = spec.layers[i]
        # dW[out,in] = dZ^T . X   (PERMUTE of X^T.dZ absorbed)
        if fuse_update:
            pb.gemm_update(dz[i], acts[i], l.fan_out, l.fan_in, batch, lay.counter,
                           (lay.weights[i], lay.first[i] if has_first else None,
                            lay.second[i] if lay.second else None, lay.weights_next[i],
                            lay.first_next[i] if has_first else None,
                            lay.second_next[i] if lay.second else None),
                           kind=kind, trans_a=True, **common)
        else:
            pb.gemm(dz[i], acts[i], gW[i], l.fan_out, l.fan_in, batch, trans_a=True)
        if gb[i] is not None and not db_fused[i]:
            pb.colsum(dz[i], gb[i], batch, l.fan_out)
    if head_loss is not None:
        pb.ce_head_loss(*head_loss)  # nothing waits on the objective but the commit
    if mode != GradientMode.RESET_AND_STEP:
        # G = accumulator + G for every tensor, each candidate checked finite
        acc_entries = [(g, g, a, None, g.count) for g, a in zip(lay.grads, lay.accum)]
        for i in range(0, len(acc_entries), 16):
            pb.optimizer(lay.counter, acc_entries[i:i + 16], kind="acc_sum", phase=0, lr=0.0)
        if mode == GradientMode.ACCUMULATE:
            for i in range(0, len(acc_entries), 16):
                pb.optimizer(lay.counter, acc_entries[i:i + 16], kind="acc_commit", phase=1, lr=0.0)
            return pb, lay
    # one staged pass: current set -> candidate set, failures flagged; then the counter
    params_next = lay.weights_next + [b for b in lay.biases_next if b is not None]
    entries = []
    for j, p in enumerate(params):
        if fuse_update and j < L:
            continue  # weight updated in its gradient GEMM's epilogue
        entries.append((p, lay.grads[j], lay.first[j] if has_first else None,
                        lay.second[j] if lay.second else None, params_next[j],
                        lay.first_next[j] if has_first else None,
                        lay.second_next[j] if lay.second else None, p.count))
    for i in range(0, len(entries), 16):
        pb.optimizer(lay.counter, entries[i:i + 16], kind=kind, phase=2, **common)
    if uses_acc:
        acc_entries = [(g, g, a, None, g.count) for g, a in zip(lay.grads, lay.accum)]
        for i in range(0, len(acc_entries), 16):
            pb.optimizer(lay.counter, acc_entries[i:i + 16], kind="acc_clear", phase=1, lr=0.0)
    pb.step_commit(lay.counter)
    return pb, lay


def lower_forward(spec: MlpSpec, batch: int):
    """Inference program (Model.compute): inputs W_1..W_L, b_1..b_L, x; output prediction."""
    pb = ProgramBuilder()
    Ws = [pb.input(l.fan_in * l.fan_out) for l in spec.layers]
    bs = [pb.input(l.fan_out) if l.bias else None for l in spec.layers]
    x = pb.input(batch * spec.layers[0].fan_in)
    out = pb.output(batch * spec.layers[-1].fan_out)
    cur = x
    for i, l in enumerate(spec.layers):
        dst = out if i == len(spec.layers) - 1 else pb.internal(batch * l.fan_out)
        pb.gemm(cur, Ws[i], dst, batch, l.fan_out, l.fan_in, trans_b=True, bias=bs[i],
                act=l.activation)
        cur = dst
    return pb


# ---- session ----
@dataclass
class TrainingStep:
    objective: float
    optimizer_step: int | None
    accumulated_gradient_runs: int = 0


@dataclass
class TrainingState:
    """Byte-exact snapshot: parameters, first/second moment slots, accumulators, counters."""
    weights: list[np.ndarray]
    biases: list[np.ndarray]
    first: list[np.ndarray]
    second: list[np.ndarray]
    optimizer_steps: int
    accumulators: list[np.ndarray] = field(default_factory=list)
    accumulated_gradient_runs: int = 0


def check_batch(spec: MlpSpec, batch: int, label_dtype: str, x, y) -> tuple[np.ndarray, np.ndarray]:
    """The host batch (x, y) as a training program's contiguous input arrays, or ValueError
    when its shape or label type does not match: x must be [batch, fan_in]; y [batch, fan_out]
    for MSE, or [batch] integer class indices for cross-entropy (INT32 labels must fit 32 bits).
    The reference rejects a mismatched input before any work (TrainingSession.java:579-647), so
    a rejected batch is never uploaded."""
    x = np.asarray(x)
    y = np.asarray(y)
    fan_in = spec.layers[0].fan_in
    fan_out = spec.layers[-1].fan_out

    def numeric(a):
        return np.issubdtype(a.dtype, np.floating) or np.issubdtype(a.dtype, np.integer)

    if x.shape != (batch, fan_in):
        raise ValueError(f"input shape {x.shape} does not match the session's ({batch}, {fan_in})")
    if not numeric(x):
        raise ValueError(f"input dtype {x.dtype} is not numeric")
    if spec.loss == "mse":
        if y.shape != (batch, fan_out):
            raise ValueError(f"target shape {y.shape} does not match the session's "
                             f"({batch}, {fan_out})")
        if not numeric(y):
            raise ValueError(f"target dtype {y.dtype} is not numeric")
        ydt = np.float32
    else:
        if y.shape != (batch,):
            raise ValueError(f"label shape {y.shape} does not match the session's ({batch},)")
        if not np.issubdtype(y.dtype, np.integer):
            raise ValueError(f"labels must be integer class indices, not {y.dtype}")
        if label_dtype == "i32":
            if y.size and (int(y.min()) < -2**31 or int(y.max()) >= 2**31):
                raise ValueError("a label does not fit the session's INT32 label type")
            ydt = np.int32
        else:
            if y.dtype == np.uint64 and y.size and int(y.max()) >= 2**63:
                raise ValueError("a label does not fit the session's INT64 label type")
            ydt = np.int64
    return np.ascontiguousarray(x, np.float32), np.ascontiguousarray(y, ydt)


class HipTrainingSession:
    """A prepared, device-resident training step (TrainingSession analogue).

    Parameters and optimizer slots live in two device buffer sets; a step reads the current set
    and writes the other, and the session adopts the written set only when the run succeeds."""

    def __init__(self, ctx: HipContext, spec: MlpSpec, weights, biases, optimizer, batch: int,
                 *, label_dtype: str = "i64"):
        self.ctx = ctx
        self.spec = spec
        self.batch = batch
        self.optimizer = optimizer
        self.label_dtype = label_dtype
        self._programs: dict[tuple, tuple[HipProgram, TrainingLayout]] = {}
        self._bindings: dict[tuple, object] = {}  # prepared handle arrays of the plain step
        self.program, lay = self._program(GradientMode.RESET_AND_STEP, False)
        self.layout = lay
        Ws = [np.asarray(w, np.float32) for w in weights]
        bs = [np.asarray(b, np.float32) for b, l in zip(biases, spec.layers) if l.bias]
        self._sets = []
        for _ in range(2):
            W = [ctx.upload(w) for w in Ws]
            b = [ctx.upload(x) for x in bs]
            params = W + b
            first = [ctx.upload(np.zeros(p.nbytes // 4, np.float32)) for p in params] if lay.first else []
            second = [ctx.upload(np.zeros(p.nbytes // 4, np.float32)) for p in params] if lay.second else []
            self._sets.append((W, b, first, second))
        self._cur = 0
        self.accum: list[HipBuffer] = []
        self.accumulated_gradient_runs = 0
        self.counter = ctx.upload(np.zeros(1, np.int64))
        self.loss = ctx.buffer(4)
        self._x = ctx.buffer(lay.x.nbytes)
        self._y = ctx.buffer(lay.y.nbytes)
        self._x2 = self._y2 = None  # second batch buffers of run_pipelined, made on first use

    @classmethod
    def open(cls, ctx, spec, weights, biases, optimizer, batch, **kw) -> "HipTrainingSession":
        return cls(ctx, spec, weights, biases, optimizer, batch, **kw)

    # current set views
    @property
    def W(self):
        return self._sets[self._cur][0]

    @property
    def b(self):
        return self._sets[self._cur][1]

    @property
    def first(self):
        return self._sets[self._cur][2]

    @property
    def second(self):
        return self._sets[self._cur][3]

    def _program(self, mode: str, clear: bool):
        key = (mode, clear)
        if key not in self._programs:
            pb, lay = lower_training_step(self.spec, self.batch, self.optimizer,
                                          label_dtype=self.label_dtype, mode=mode,
                                          clear_accumulator=clear)
            self._programs[key] = (HipProgram(self.ctx, pb.image()), lay)
        return self._programs[key]

    def _ensure_accumulators(self):
        if not self.accum:
            self.accum = [self.ctx.upload(np.zeros(p.nbytes // 4, np.float32)) for p in self.W + self.b]

    def run_resident(self, x: HipBuffer, y: HipBuffer,
                     mode: str = GradientMode.RESET_AND_STEP) -> None:
        """One run on device-resident batch buffers; the objective stays on the device."""
        pending = self.accumulated_gradient_runs > 0
        if mode == GradientMode.RESET_AND_STEP and not pending:
            # the plain step: its two handle arrays (one per current set) are built once per
            # batch buffer pair
            key = (self._cur, x.handle.value, y.handle.value)
            bound = self._bindings.get(key)
            prog, _ = self._programs[(mode, False)]
            if bound is None:
                cur, nxt = self._sets[self._cur], self._sets[1 - self._cur]
                bound = prog.bind(cur[0] + cur[1] + cur[2] + cur[3] + nxt[0] + nxt[1] + nxt[2]
                                  + nxt[3] + [self.counter, x, y], [self.loss])
                if len(self._bindings) >= 8:
                    self._bindings.clear()
                self._bindings[key] = bound
            prog.run_bound(bound)
            self._cur = 1 - self._cur
            return
        cur = self._sets[self._cur]
        nxt = self._sets[1 - self._cur]
        current = cur[0] + cur[1] + cur[2] + cur[3]
        candidate = nxt[0] + nxt[1] + nxt[2] + nxt[3]
        self._ensure_accumulators()
        prog, _ = self._program(mode, mode == GradientMode.RESET_AND_STEP)
        if mode == GradientMode.ACCUMULATE:
            prog.run(current + self.accum + [self.counter, x, y], [self.loss])
            self.accumulated_gradient_runs += 1
            return
        prog.run(current + candidate + self.accum + [self.counter, x, y], [self.loss])
        # reached only when the program committed
        self._cur = 1 - self._cur
        self.accumulated_gradient_runs = 0

    def _checked_batch(self, x, y) -> tuple[np.ndarray, np.ndarray]:
        return check_batch(self.spec, self.batch, self.label_dtype, x, y)

    def run(self, x: np.ndarray, y: np.ndarray,
            mode: str = GradientMode.RESET_AND_STEP) -> TrainingStep:
        """Uploads the batch (borrow), runs once in `mode`, downloads the objective. A batch
        whose shape or label type differs from the session's raises ValueError and changes
        no state."""
        x, y = self._checked_batch(x, y)
        self._x.upload(x)
        self._y.upload(y)
        self.run_resident(self._x, self._y, mode)
        step = None if mode == GradientMode.ACCUMULATE else self.optimizer_steps
        return TrainingStep(float(self.objective()), step, self.accumulated_gradient_runs)

    def run_pipelined(self, batches, mode: str = GradientMode.RESET_AND_STEP) -> list:
        """One run per (x, y) host batch of `batches`, each step's batch uploaded through the
        context's pinned staging ring on its copy stream while the previous step runs
        (`shk_hip_buffer_upload_staged`, `shk_hip_program_run_async`), into two alternating
        batch buffers. Results, state and failure behaviour are those of calling `run` once per
        batch: every batch's shape is checked before the first run (ValueError, no state
        changed), a failed step raises, commits nothing, and no later step runs. RESET_AND_STEP
        without pending accumulated gradients is pipelined; other cases run step by step."""
        checked = [self._checked_batch(x, y) for x, y in batches]
        if mode != GradientMode.RESET_AND_STEP or self.accumulated_gradient_runs > 0:
            return [self.run(x, y, mode) for x, y in checked]
        if not checked:
            return []
        if self._x2 is None:
            self._x2 = self.ctx.buffer(self._x.nbytes)
            self._y2 = self.ctx.buffer(self._y.nbytes)
        xs, ys = (self._x, self._x2), (self._y, self._y2)
        xs[0].upload_staged(checked[0][0])
        ys[0].upload_staged(checked[0][1])
        prog, _ = self._programs[(mode, False)]
        # One stream while batches stream in: kernels on the second compute stream slow the
        # staged copies (measured on the MLP-4096 step: 14.0 ms per step with one stream,
        # 15.0 ms with two), and steps large enough to make the upload worth hiding fill the
        # GPU without it. The two-stream schedule comes back afterwards.
        was_concurrent = prog.side_steps() > 0
        prog.set_concurrent(False)
        try:
            return self._pipelined_steps(prog, checked, xs, ys)
        finally:
            if was_concurrent:
                prog.set_concurrent(True)

    def _pipelined_steps(self, prog, checked, xs, ys) -> list:
        steps = []
        for i in range(len(checked)):
            slot = i & 1
            cur = self._sets[self._cur]
            cand = self._sets[1 - self._cur]
            prog.run_async(cur[0] + cur[1] + cur[2] + cur[3] + cand[0] + cand[1] + cand[2] + cand[3]
                           + [self.counter, xs[slot], ys[slot]], [self.loss])
            try:
                if i + 1 < len(checked):  # overlaps the run just enqueued
                    xs[1 - slot].upload_staged(checked[i + 1][0])
                    ys[1 - slot].upload_staged(checked[i + 1][1])
            finally:
                # Completes the pending run even when staging raised: a run that succeeded has
                # committed on the device, so the session adopts its candidate set before the
                # staging error propagates; a failed run raises here and commits nothing.
                prog.wait()
                self._cur = 1 - self._cur
            steps.append(TrainingStep(float(self.objective()), self.optimizer_steps, 0))
        return steps

    def zero_grad(self) -> None:
        """Empties the pending gradient accumulator (TrainingSession.zeroGrad)."""
        for a in self.accum:
            a.upload(np.zeros(a.nbytes // 4, np.float32))
        self.accumulated_gradient_runs = 0

    def objective(self) -> np.float32:
        return self.loss.download(np.float32, 1)[0]

    @property
    def optimizer_steps(self) -> int:
        return int(self.counter.download(np.int64, 1)[0])

    def state(self) -> TrainingState:
        return TrainingState(
            [w.download().reshape(l.fan_out, l.fan_in) for w, l in zip(self.W, self.spec.layers)],
            [b.download() for b in self.b],
            [m.download() for m in self.first],
            [v.download() for v in self.second],
            self.optimizer_steps,
            [a.download() for a in self.accum] if self.accumulated_gradient_runs else [],
            self.accumulated_gradient_runs)

    def restore(self, st: TrainingState) -> None:
        for buf, a in zip(self.W, st.weights):
            buf.upload(np.asarray(a, np.float32))
        for buf, a in zip(self.b, st.biases):
            buf.upload(np.asarray(a, np.float32))
        for buf, a in zip(self.first, st.first):
            buf.upload(np.asarray(a, np.float32))
        for buf, a in zip(self.second, st.second):
            buf.upload(np.asarray(a, np.float32))
        self.counter.upload(np.array([st.optimizer_steps], np.int64))
        if st.accumulated_gradient_runs:
            self._ensure_accumulators()
            for buf, a in zip(self.accum, st.accumulators):
                buf.upload(np.asarray(a, np.float32))
        else:
            self.zero_grad()
        self.accumulated_gradient_runs = st.accumulated_gradient_runs

    def close(self) -> None:
        self._bindings.clear()
        for prog, _ in self._programs.values():
            prog.close()
        self._programs.clear()


def lower_dense_layer(batch: int, fan_in: int, fan_out: int, activation: str | None = "relu",
                      weight_layout: str = "in_out"):
    """One fused layer forward + backward with an upstream cotangent (benchmark configuration C2):
    Y = act(X . W + b) for W [in, out] (weight_layout "in_out", the config's X.W) or
    Y = act(X . W^T + b) for W [out, in] ("out_in", Linear's layout); returns Y, dX, dW, db.

    Inputs X [B,in], W, b [out], dY [B,out]; outputs Y, dX [B,in], dW (W's layout), db [out].
    The forward GEMM's epilogue also forms dZ = act_grad(dY, Y) and the column sums db of dZ;
    dX and dW are MFMA GEMMs over dZ.
    """
    from .program import PW
    pb = ProgramBuilder()
    X = pb.input(batch * fan_in)
    W = pb.input(fan_in * fan_out)
    b = pb.input(fan_out)
    dY = pb.input(batch * fan_out)
    Y = pb.output(batch * fan_out)
    dX = pb.output(batch * fan_in)
    dW = pb.output(fan_in * fan_out)
    db = pb.output(fan_out)
    in_out = weight_layout == "in_out"
    if activation is None:
        # dZ = dY: the backward GEMMs read the cotangent as given
        pb.gemm(X, W, Y, batch, fan_out, fan_in, trans_b=not in_out, bias=b)
        dZ = dY
        pb.colsum(dZ, db, batch, fan_out)
    else:
        # the forward GEMM's epilogue also forms dZ = act_grad(dY, Y) and db = SUM_TO_SHAPE(dZ)
        dZ = pb.internal(batch * fan_out)
        pb.gemm(X, W, Y, batch, fan_out, fan_in, trans_b=not in_out, bias=b, act=activation,
                dy=dY, dz=dZ, colsum=db)
    if in_out:
        pb.gemm(dZ, W, dX, batch, fan_in, fan_out, trans_b=True)        # dX = dZ . W^T
        pb.gemm(X, dZ, dW, fan_in, fan_out, batch, trans_a=True)        # dW = X^T . dZ
    else:
        pb.gemm(dZ, W, dX, batch, fan_in, fan_out)                      # dX = dZ . W
        pb.gemm(dZ, X, dW, fan_out, fan_in, batch, trans_a=True)        # dW = dZ^T . X
    return pb, (Y, dX, dW, db)
