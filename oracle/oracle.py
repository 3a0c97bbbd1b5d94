"""numpy/ctypes front end of the CPU oracle (liboracle_synaptik.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg as the checker / the timed CPU restatement; never by the synaptik_amd product.

Every function restates a reference algorithm (citations in synaptik_oracle.c). The MLP
training step composes them exactly as the reference's compiled graph does:
  forward  Y_l = act_l(X_l . W_l^T + b_l)          (TensorLinearExpressions.java:97-146)
  loss     MSE MEAN or index categorical CE MEAN  (CpuLossReferenceKernel.java)
  backward dW_l = PERMUTE(X_l^T . dZ_l), db_l = SUM_TO_SHAPE(dZ_l), dX_l = dZ_l . W_l,
           dZ_{l-1} = act_grad(dX_l, Y_{l-1})      (LinearAlgebraGradientRules.java:97-104,
                                                   ElementwiseGradientRules.java:99-105,205-210)
  update   SGD / Adam / AdamW, staged for every tensor and committed only if all stages pass
           (TrainingParameter.java:433-525,622-672; TrainingSession.java:579-647).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_synaptik.so"

_lib = None

F32P = ctypes.POINTER(ctypes.c_float)
I64P = ctypes.POINTER(ctypes.c_int64)
i64 = ctypes.c_int64
i32 = ctypes.c_int
f32 = ctypes.c_float

ACT = {None: 0, "none": 0, "relu": 1, "tanh": 2, "sigmoid": 3}


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle_synaptik.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        sigs = {
            "shko_matmul_f32": (None, [F32P, F32P, F32P, i64, i64, i64, i64, i64, i64, i32, i32]),
            "shko_exact_sum": (f32, [F32P, i64, i64]),
            "shko_exact_mean": (f32, [F32P, i64, i64]),
            "shko_exact_quotient": (f32, [f32, i64]),
            "shko_max": (f32, [F32P, i64, i64]),
            "shko_colsum": (None, [F32P, F32P, i64, i64, i64]),
            "shko_activation": (None, [i32, F32P, F32P, i64]),
            "shko_activation_grad": (None, [i32, F32P, F32P, F32P, i64]),
            "shko_linear_forward": (None, [F32P, F32P, F32P, F32P, i64, i64, i64, i32]),
            "shko_softmax_rows": (None, [F32P, F32P, i64, i64, i32]),
            "shko_logsumexp_rows": (None, [F32P, F32P, i64, i64]),
            "shko_softmax_grad_rows": (None, [F32P, F32P, F32P, i64, i64]),
            "shko_logsumexp_grad_rows": (None, [F32P, F32P, F32P, F32P, i64, i64]),
            "shko_mse_mean": (f32, [F32P, F32P, i64]),
            "shko_mse_sum": (f32, [F32P, F32P, i64]),
            "shko_mse_mean_exact": (f32, [F32P, F32P, i64]),
            "shko_mse_grad": (None, [F32P, F32P, F32P, i64, f32, i32]),
            "shko_index_ce_mean": (i32, [F32P, I64P, i64, i64, i32, i64, F32P]),
            "shko_index_ce_grad": (None, [F32P, I64P, F32P, i64, i64, i32, i64, f32]),
            "shko_sgd_stage": (i32, [F32P, F32P, F32P, F32P, F32P, i64, f32, f32, f32, f32, i32,
                                     i32, i64]),
            "shko_adam_stage": (i32, [F32P, F32P, F32P, F32P, F32P, F32P, F32P, i64, f32, f32,
                                      f32, f32, f32, i32, i64]),
            "shko_adam_apply": (i32, [F32P, F32P, F32P, F32P, i64, f32, f32, f32, f32, f32, i32, i64]),
            "shko_canonical_bytes": (i32, [ctypes.c_void_p, ctypes.c_uint64, i32, i32, i32, I64P,
                                           I64P, i64, ctypes.c_void_p]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(F32P)


def _c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- primitives ----
def matmul(A, B, trans_a=False, trans_b=False) -> np.ndarray:
    A, B = _c(A), _c(B)
    M, K = (A.shape[1], A.shape[0]) if trans_a else A.shape
    N = B.shape[0] if trans_b else B.shape[1]
    C = np.empty((M, N), np.float32)
    lib().shko_matmul_f32(_f(A), _f(B), _f(C), M, N, K, A.shape[1], B.shape[1], N,
                          int(trans_a), int(trans_b))
    return C


def exact_sum(x) -> np.float32:
    x = _c(x).ravel()
    return np.float32(lib().shko_exact_sum(_f(x), x.size, 1))


def exact_mean(x) -> np.float32:
    x = _c(x).ravel()
    return np.float32(lib().shko_exact_mean(_f(x), x.size, 1))


def max_reduce(x) -> np.float32:
    """MAX over every element of x (Java Math.max fold, AggregateReductionKind.java:128-137)."""
    x = _c(x).ravel()
    return np.float32(lib().shko_max(_f(x), x.size, 1))


def max_rows(X) -> np.ndarray:
    X = _c(X)
    return np.array([lib().shko_max(_f(X[r]), X.shape[1], 1) for r in range(X.shape[0])],
                    np.float32)


def exact_quotient(value, count) -> np.float32:
    return np.float32(lib().shko_exact_quotient(float(np.float32(value)), int(count)))


def colsum(X) -> np.ndarray:
    X = _c(X)
    out = np.empty(X.shape[1], np.float32)
    lib().shko_colsum(_f(X), _f(out), X.shape[0], X.shape[1], X.shape[1])
    return out


def activation(act, x) -> np.ndarray:
    x = _c(x)
    y = np.empty_like(x)
    lib().shko_activation(ACT[act], _f(x), _f(y), x.size)
    return y


def activation_grad(act, g, y) -> np.ndarray:
    g, y = _c(g), _c(y)
    d = np.empty_like(g)
    lib().shko_activation_grad(ACT[act], _f(g), _f(y), _f(d), g.size)
    return d


def linear_forward(X, W, b, act=None) -> np.ndarray:
    X, W = _c(X), _c(W)
    Bn, fin = X.shape
    fout = W.shape[0]
    Y = np.empty((Bn, fout), np.float32)
    bp = _f(_c(b)) if b is not None else None
    lib().shko_linear_forward(_f(X), _f(W), bp, _f(Y), Bn, fin, fout, ACT[act])
    return Y


def softmax_rows(X, log=False) -> np.ndarray:
    X = _c(X)
    Y = np.empty_like(X)
    lib().shko_softmax_rows(_f(X), _f(Y), X.shape[0], X.shape[1], int(log))
    return Y


def logsumexp_rows(X) -> np.ndarray:
    X = _c(X)
    out = np.empty(X.shape[0], np.float32)
    lib().shko_logsumexp_rows(_f(X), _f(out), X.shape[0], X.shape[1])
    return out


def softmax_grad_rows(Y, G) -> np.ndarray:
    Y, G = _c(Y), _c(G)
    D = np.empty_like(Y)
    lib().shko_softmax_grad_rows(_f(Y), _f(G), _f(D), Y.shape[0], Y.shape[1])
    return D


def logsumexp_grad_rows(X, lse, g) -> np.ndarray:
    X, lse, g = _c(X), _c(lse), _c(g)
    D = np.empty_like(X)
    lib().shko_logsumexp_grad_rows(_f(X), _f(lse), _f(g), _f(D), X.shape[0], X.shape[1])
    return D


def mse_mean(p, t) -> np.float32:
    p, t = _c(p).ravel(), _c(t).ravel()
    return np.float32(lib().shko_mse_mean(_f(p), _f(t), p.size))


def mse_mean_exact(p, t) -> np.float32:
    """MSE MEAN with the contract's exact reduction (shko_mse_mean_exact)."""
    p, t = _c(p).ravel(), _c(t).ravel()
    return np.float32(lib().shko_mse_mean_exact(_f(p), _f(t), p.size))


def mse_sum(p, t) -> np.float32:
    p, t = _c(p).ravel(), _c(t).ravel()
    return np.float32(lib().shko_mse_sum(_f(p), _f(t), p.size))


def mse_grad(p, t, g=1.0, reduction="mean") -> np.ndarray:
    p, t = _c(p), _c(t)
    d = np.empty_like(p)
    lib().shko_mse_grad(_f(p), _f(t), _f(d), p.size, float(g), int(reduction == "sum"))
    return d


def index_ce_mean(logits, target, ignore_index=None) -> np.float32:
    logits = _c(logits)
    t = np.ascontiguousarray(target, dtype=np.int64)
    out = ctypes.c_float()
    rc = lib().shko_index_ce_mean(_f(logits), t.ctypes.data_as(I64P), logits.shape[0], logits.shape[1],
                                  0 if ignore_index is None else 1,
                                  0 if ignore_index is None else int(ignore_index),
                                  ctypes.byref(out))
    if rc != 0:
        raise ValueError("index target out of bounds")
    return np.float32(out.value)


def index_ce_grad(logits, target, ignore_index=None, g=1.0) -> np.ndarray:
    logits = _c(logits)
    t = np.ascontiguousarray(target, dtype=np.int64)
    d = np.empty_like(logits)
    lib().shko_index_ce_grad(_f(logits), t.ctypes.data_as(I64P), _f(d), logits.shape[0],
                             logits.shape[1], 0 if ignore_index is None else 1,
                             0 if ignore_index is None else int(ignore_index), float(g))
    return d


def sgd_stage(p, g, m, *, lr, momentum=0.0, dampening=0.0, weight_decay=0.0, nesterov=False,
              has_momentum_slot=None, completed_steps=0):
    """Returns (p_candidate, m_candidate) or raises ArithmeticError."""
    p, g = _c(p), _c(g)
    m = _c(m) if m is not None else np.zeros_like(p)
    if has_momentum_slot is None:
        has_momentum_slot = momentum != 0.0
    pc, mc = p.copy(), m.copy()
    rc = lib().shko_sgd_stage(_f(p), _f(g), _f(m), _f(pc), _f(mc), p.size, lr, momentum, dampening,
                              weight_decay, int(nesterov), int(has_momentum_slot), int(completed_steps))
    if rc:
        raise ArithmeticError("SGD intermediate or candidate is not finite")
    return pc, mc


def adam_stage(p, g, m, v, *, lr, beta1, beta2, eps, weight_decay=0.0, decoupled=False,
               completed_steps=0):
    p, g, m, v = _c(p), _c(g), _c(m), _c(v)
    pc, mc, vc = p.copy(), m.copy(), v.copy()
    rc = lib().shko_adam_stage(_f(p), _f(g), _f(m), _f(v), _f(pc), _f(mc), _f(vc), p.size, lr, beta1,
                               beta2, eps, weight_decay, int(decoupled), int(completed_steps))
    if rc:
        raise ArithmeticError("Adam intermediate or candidate is not finite")
    return pc, mc, vc


def adam_apply(p, m_new, v_new, *, lr, beta1, beta2, eps, weight_decay=0.0, decoupled=False,
               completed_steps=0):
    """Adam's parameter candidates from given new moments (the arithmetic after the moment
    updates in stageAdaptiveElement32, TrainingParameter.java:433-525)."""
    p, m_new, v_new = _c(p), _c(m_new), _c(v_new)
    pc = p.copy()
    rc = lib().shko_adam_apply(_f(p), _f(m_new), _f(v_new), _f(pc), p.size, lr, beta1, beta2,
                               eps, weight_decay, int(decoupled), int(completed_steps))
    if rc:
        raise ArithmeticError("Adam intermediate or candidate is not finite")
    return pc


# ---- MLP training step ----
def canonical_bytes(raw: bytes, width: int, shape, strides=None, offset: int = 0,
                    boolean: bool = False) -> bytes:
    """Canonical big-endian row-major bytes of a view over little-endian storage `raw`
    (MetalBackendRuntime.java:360-398,489-499). Raises ValueError for a non-canonical BOOL byte
    or a view outside the storage."""
    shape = tuple(int(d) for d in shape)
    count = int(np.prod(shape, dtype=np.int64)) if shape else 1
    w = 1 if boolean else int(width)
    src = np.frombuffer(bytes(raw), dtype=np.uint8)
    dst = np.zeros(max(1, count * w), np.uint8)
    dims = (ctypes.c_int64 * max(1, len(shape)))(*shape)
    st = None if strides is None else (ctypes.c_int64 * max(1, len(shape)))(*strides)
    rc = lib().shko_canonical_bytes(src.ctypes.data if src.size else None, src.size, w,
                                    1 if boolean else 0, len(shape), dims, st, int(offset),
                                    dst.ctypes.data)
    if rc == 1:
        raise ValueError("BOOL source contains a non-canonical byte")
    if rc == 2:
        raise ValueError("view lies outside the storage")
    return dst.tobytes()[:count * w]


_LONG_MIN, _LONG_MAX = -(1 << 63), (1 << 63) - 1


def _exact(v: int) -> int:
    """Java Math.*Exact: a result outside the signed 64-bit range throws ArithmeticException."""
    if not _LONG_MIN <= v <= _LONG_MAX:
        raise ArithmeticError("long overflow")
    return v


def storage_transfer_bytes(width: int, shape, strides, offset: int) -> int:
    """Byte extent of a prepared storage-layout transfer, or 0 when the view is not one.

    Restates MetalBackendRuntime.isStorageTransfer / transferByteCount
    (modules/backend/metal/.../MetalBackendRuntime.java:425-484) and
    CpuMetalPreparedBufferTransfer.transferByteCount (modules/engine/.../
    CpuMetalPreparedBufferTransfer.java:79-127): rank <= 16, every extent and stride > 0, the
    axes of extent > 1 insertion-sorted by stride (only a strictly larger stride moves ahead),
    each stride >= the span covered so far (covered starts at 1 and grows by (extent - 1) *
    stride), referencedElementSpan = offset + covered (LayoutGeometry.referencedElementSpan for a
    non-empty view), and span * width a positive long. Any Math.*Exact overflow rejects.
    `strides` None is the contiguous row-major layout (LayoutDescriptor.contiguous)."""
    shape = [int(d) for d in shape]
    if len(shape) > 16 or width not in (1, 2, 4, 8) or offset < 0:
        return 0
    if strides is None:
        strides, e = [0] * len(shape), 1
        for a in range(len(shape) - 1, -1, -1):
            strides[a] = e
            e *= max(shape[a], 1)
    strides = [int(x) for x in strides]
    act_s, act_d = [], []
    try:
        for d, st in zip(shape, strides):
            if d <= 0 or st <= 0:
                return 0
            _exact(d)
            _exact(st)
            if d > 1:
                i = len(act_s)
                act_s.append(st)
                act_d.append(d)
                while i > 0 and act_s[i - 1] > st:
                    act_s[i], act_d[i] = act_s[i - 1], act_d[i - 1]
                    i -= 1
                act_s[i], act_d[i] = st, d
        covered = 1
        for st, d in zip(act_s, act_d):
            if st < covered:
                return 0
            covered = _exact(covered + _exact((d - 1) * st))
        span = _exact(int(offset) + covered)
        nbytes = _exact(span * width)
    except ArithmeticError:
        return 0
    return nbytes if nbytes > 0 else 0


class OracleMLP:
    """Fully-connected network with per-layer activations; weights W[out,in], biases [out].

    loss: "mse" (prediction vs float target) or "ce" (index categorical CE over logits).
    optimizer: dict(kind="sgd", lr, momentum, dampening, weight_decay, nesterov) or
               dict(kind="adam"/"adamw", lr, beta1, beta2, eps, weight_decay).
    """

    def __init__(self, weights, biases, acts, loss, optimizer, reduction="mean", gemm="oracle",
                 mse_sum="sequential"):
        self.W = [np.array(w, np.float32) for w in weights]
        self.b = [np.array(b, np.float32) for b in biases if b is not None]
        self.has_bias = [b is not None for b in biases]
        self.acts = list(acts)
        self.loss = loss
        self.reduction = reduction
        self.opt = dict(optimizer)
        self.m = [np.zeros_like(w) for w in self.W] + [np.zeros_like(b) for b in self.b]
        self.v = [np.zeros_like(w) for w in self.W] + [np.zeros_like(b) for b in self.b]
        self.steps = 0
        # "oracle": the reference's sequential no-FMA GEMM (shko_matmul_f32); "float64": every
        # GEMM evaluated in binary64 (numpy) and rounded once to binary32, for network sizes the
        # scalar GEMM cannot finish in a test's time. All other operations are the oracle's.
        if gemm not in ("oracle", "float64"):
            raise ValueError(gemm)
        self.gemm = gemm
        # "sequential": the reference CPU kernels' binary32 running sum of the squares;
        # "exact": the Model contract's exact reduction (mse_mean_exact). MEAN reduction only.
        if mse_sum not in ("sequential", "exact"):
            raise ValueError(mse_sum)
        self.mse_sum = mse_sum

    def _mm(self, A, B, trans_a=False, trans_b=False):
        if self.gemm == "oracle":
            return matmul(A, B, trans_a=trans_a, trans_b=trans_b)
        a = A.astype(np.float64)
        b = B.astype(np.float64)
        return np.ascontiguousarray((a.T if trans_a else a) @ (b.T if trans_b else b),
                                    dtype=np.float32)

    def forward(self, x):
        xs = [_c(x)]
        bi = iter(self.b)
        for W, hb, a in zip(self.W, self.has_bias, self.acts):
            b = next(bi) if hb else None
            if self.gemm == "oracle":
                xs.append(linear_forward(xs[-1], W, b, a))
            else:  # Z = X.W^T rounded, then + b in binary32, then the activation
                z = self._mm(xs[-1], W, trans_b=True)
                if b is not None:
                    z = (z + b[None, :]).astype(np.float32)
                xs.append(activation(a, z) if a else z)
        return xs

    def gradients(self, x, y):
        xs = self.forward(x)
        pred = xs[-1]
        if self.loss == "mse":
            if self.reduction == "mean":
                loss = mse_mean_exact(pred, y) if self.mse_sum == "exact" else mse_mean(pred, y)
            else:
                loss = mse_sum(pred, y)
            dz = mse_grad(pred, y, reduction=self.reduction)
        else:
            loss = index_ce_mean(pred, y)
            dz = index_ce_grad(pred, y)
        L = len(self.W)
        gW, gb = [None] * L, [None] * L
        self.last_cotangents = [None] * L  # dZ_l of the last gradients() call, per layer
        for l in reversed(range(L)):
            self.last_cotangents[l] = dz
            gW[l] = self._mm(dz, xs[l], trans_a=True)
            gb[l] = colsum(dz) if self.has_bias[l] else None
            if l > 0:
                dx = self._mm(dz, self.W[l])
                dz = activation_grad(self.acts[l - 1], dx, xs[l])
        return loss, gW, gb, xs

    def step(self, x, y):
        """One training step; returns the objective. Raises ArithmeticError without commit."""
        loss, gW, gb, xs = self.gradients(x, y)
        self.last_inputs, self.last_gradients = xs, gW + [g for g in gb if g is not None]
        params = self.W + self.b
        grads = gW + [g for g in gb if g is not None]
        o = self.opt
        staged = []
        for i, (p, g) in enumerate(zip(params, grads)):
            if o["kind"] == "sgd":
                pc, mc = sgd_stage(p, g, self.m[i], lr=o["lr"], momentum=o.get("momentum", 0.0),
                                   dampening=o.get("dampening", 0.0),
                                   weight_decay=o.get("weight_decay", 0.0),
                                   nesterov=o.get("nesterov", False), completed_steps=self.steps)
                staged.append((pc, mc, self.v[i]))
            else:
                pc, mc, vc = adam_stage(p, g, self.m[i], self.v[i], lr=o["lr"], beta1=o["beta1"],
                                        beta2=o["beta2"], eps=o["eps"],
                                        weight_decay=o.get("weight_decay", 0.0),
                                        decoupled=o["kind"] == "adamw", completed_steps=self.steps)
                staged.append((pc, mc, vc))
        L = len(self.W)
        for i, (pc, mc, vc) in enumerate(staged):
            if i < L:
                self.W[i] = pc
            else:
                self.b[i - L] = pc
            self.m[i] = mc
            self.v[i] = vc
        self.steps += 1
        return loss
