"""Seeded parameter initialization, mirroring the reference's initializer surface.

* `ParameterInitializers` (extensions/nn/.../initialization/ParameterInitializers.java): zeros,
  ones, normal, uniform, glorot_normal, glorot_uniform, kaiming_relu_normal,
  kaiming_relu_uniform and `initialize(shape, policy, source)`, with the reference's validation
  order, fan convention (weight shape [fanOut, fanIn]: fanOut = dim 0, fanIn = dim 1,
  :380-402), bounds computed in binary64 (:269-372), one draw per element in row-major order,
  and each draw narrowed once to the element type (TensorRandoms.java:615-629,783-796).
* Random sources are pluggable: anything with `next_double(origin, bound)` and/or
  `next_gaussian()` (the two RandomGenerator methods the initializers call). Sources may also
  offer `uniform_block(origin, bound, count, dtype)` / `gaussian_block(count)` to draw many values
  in one call, with the same values as the per-element calls.
* `L64X128MixRandom(seed)`: the generator ModelBuilder and Linear use (ModelBuilder.java:74-76),
  restated natively in libsynaptik_hip.so (csrc/lxm.cpp), with `next_gaussian` as McFarland's
  modified ziggurat (the method of the JDK's RandomSupport.computeNextGaussian; tables built from
  that construction, so whether they equal the JDK's bit for bit is not checked).
* `builder_parameters(spec, seed)`: the weights and biases `Model.builder().seed(seed)` creates
  for a Linear chain: appended step i (Linear layers and activation steps both count) gets a
  fresh L64X128MixRandom(seed + 0x9E3779B97F4A7C15 * i) with long wraparound; weights are
  Glorot-uniform [out, in], biases exact zeros (ModelBuilder.java:42-45,135-137,492-494).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Sequence

import numpy as np

STEP_SEED = 0x9E3779B97F4A7C15
JAVA_ARRAY_LIMIT = 2**31 - 1
_DTYPES = {"FLOAT32": np.float32, "FLOAT64": np.float64}

_lib = None


def _native():
    global _lib
    if _lib is None:
        from .native import load_library
        L = load_library()
        u64p = ctypes.POINTER(ctypes.c_uint64)
        L.shk_lxm_seed.argtypes = [ctypes.c_int64, u64p]
        L.shk_lxm_next_long.argtypes = [u64p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_int64)]
        L.shk_lxm_next_double.argtypes = [u64p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)]
        L.shk_lxm_uniform_f64.argtypes = [u64p, ctypes.c_double, ctypes.c_double, ctypes.c_uint64,
                                          ctypes.POINTER(ctypes.c_double)]
        L.shk_lxm_uniform_f32.argtypes = [u64p, ctypes.c_double, ctypes.c_double, ctypes.c_uint64,
                                          ctypes.POINTER(ctypes.c_float)]
        L.shk_lxm_next_gaussian.argtypes = [u64p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)]
        L.shk_lxm_gaussian_tables.argtypes = [ctypes.c_uint32, ctypes.POINTER(ctypes.c_double),
                                              ctypes.POINTER(ctypes.c_double), u64p,
                                              ctypes.POINTER(ctypes.c_uint16),
                                              ctypes.POINTER(ctypes.c_uint32),
                                              ctypes.POINTER(ctypes.c_double)]
        for fn in (L.shk_lxm_seed, L.shk_lxm_next_long, L.shk_lxm_next_double,
                   L.shk_lxm_uniform_f64, L.shk_lxm_uniform_f32, L.shk_lxm_next_gaussian,
                   L.shk_lxm_gaussian_tables):
            fn.restype = ctypes.c_int32
        _lib = L
    return _lib


def _java_long(v: int) -> int:
    """v wrapped to a signed 64-bit Java long."""
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >= 1 << 63 else v


def _check_range(origin: float, bound: float) -> None:
    # RandomGenerator.nextDouble(origin, bound) range check
    if not (math.isfinite(origin) and math.isfinite(bound) and origin < bound
            and math.isfinite(bound - origin)):
        raise ValueError(f"bound must be greater than origin and the range finite: "
                         f"{origin}, {bound}")


class L64X128MixRandom:
    """java.util.random's L64X128MixRandom created from a long seed (its state: four uint64
    words advanced in place by the native restatement)."""

    def __init__(self, seed: int):
        self._state = (ctypes.c_uint64 * 4)()
        if _native().shk_lxm_seed(_java_long(int(seed)), self._state) != 0:
            raise RuntimeError("shk_lxm_seed failed")

    @property
    def state(self) -> tuple[int, int, int, int]:
        """(a, s, x0, x1)."""
        return tuple(int(v) for v in self._state)

    def next_longs(self, count: int) -> np.ndarray:
        out = np.empty(count, np.int64)
        _native().shk_lxm_next_long(self._state, count,
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)))
        return out

    def next_long(self) -> int:
        return int(self.next_longs(1)[0])

    def next_doubles(self, count: int) -> np.ndarray:
        out = np.empty(count, np.float64)
        _native().shk_lxm_next_double(self._state, count,
                                      out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
        return out

    def uniform_block(self, origin: float, bound: float, count: int, dtype) -> np.ndarray:
        """count successive nextDouble(origin, bound) draws narrowed once to dtype."""
        _check_range(origin, bound)
        if np.dtype(dtype) == np.float32:
            out = np.empty(count, np.float32)
            rc = _native().shk_lxm_uniform_f32(self._state, origin, bound, count,
                                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        else:
            out = np.empty(count, np.float64)
            rc = _native().shk_lxm_uniform_f64(self._state, origin, bound, count,
                                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
        if rc != 0:
            raise ValueError("invalid uniform range")
        return out

    def next_double(self, origin: float | None = None, bound: float | None = None) -> float:
        if origin is None:
            return float(self.next_doubles(1)[0])
        return float(self.uniform_block(origin, bound, 1, np.float64)[0])

    def gaussian_block(self, count: int) -> np.ndarray:
        """count successive nextGaussian() draws (binary64)."""
        out = np.empty(count, np.float64)
        if _native().shk_lxm_next_gaussian(self._state, count,
                                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_double))):
            raise RuntimeError("shk_lxm_next_gaussian failed")
        return out

    def next_gaussian(self) -> float:
        return float(self.gaussian_block(1)[0])


def gaussian_tables() -> dict:
    """The nextGaussian ziggurat's tables (shk_lxm_gaussian_tables): layers R, box area A, x[0..R],
    region areas (tail, overhangs, cap), alias thresholds (over 2^56) and alias columns."""
    L = _native()
    x = np.zeros(257, np.float64)
    area = np.zeros(257, np.float64)
    thr = np.zeros(256, np.uint64)
    alias = np.zeros(256, np.uint16)
    layers = ctypes.c_uint32()
    box = ctypes.c_double()
    if L.shk_lxm_gaussian_tables(257, x.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                                 area.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                                 thr.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                 alias.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                                 ctypes.byref(layers), ctypes.byref(box)):
        raise RuntimeError("shk_lxm_gaussian_tables failed")
    R = layers.value
    return dict(layers=R, box_area=box.value, x=x[:R + 1].copy(), region_area=area[:R + 1].copy(),
                threshold=thr, alias=alias)


# ---- policies (ParameterInitialization) ----
@dataclass(frozen=True)
class ParameterInitialization:
    """A closed initialization policy (ParameterInitialization.java): kind plus the two scalar
    arguments of NORMAL (mean, deviation) and UNIFORM (lower, upper)."""
    kind: str
    first: float = 0.0
    second: float = 0.0

    KINDS = ("glorot_normal", "glorot_uniform", "kaiming_relu_normal", "kaiming_relu_uniform",
             "normal", "uniform", "zeros", "ones")

    def __post_init__(self):
        if self.kind not in self.KINDS:
            raise ValueError(f"unknown initialization {self.kind}")

    @property
    def requires_random_generator(self) -> bool:
        return self.kind not in ("zeros", "ones")


def _dtype(data_type: str):
    if data_type not in _DTYPES:
        raise ValueError(f"parameter initialization requires a floating data type: {data_type}")
    return _DTYPES[data_type]


def _count(shape: Sequence[int], what: str) -> int:
    n = 1
    for d in shape:
        if d < 0:
            raise ValueError(f"{what} requires a fully static shape: {tuple(shape)}")
        n *= d
    if n > JAVA_ARRAY_LIMIT:
        raise ValueError(f"{what} element count exceeds Java array limit: required={n}, "
                         f"maximum={JAVA_ARRAY_LIMIT}")
    return n


def _uniform_draws(source, lower: float, upper: float, n: int, dt) -> np.ndarray:
    if hasattr(source, "uniform_block"):
        return source.uniform_block(lower, upper, n, dt)
    out = np.empty(n, dt)
    for i in range(n):  # one call per element, in row-major order
        out[i] = dt(source.next_double(lower, upper))
    return out


def zeros(shape, data_type: str = "FLOAT32") -> np.ndarray:
    dt = _dtype(data_type)
    _count(shape, "parameter initialization")
    return np.zeros(tuple(shape), dt)


def ones(shape, data_type: str = "FLOAT32") -> np.ndarray:
    dt = _dtype(data_type)
    _count(shape, "parameter initialization")
    return np.ones(tuple(shape), dt)


def normal(shape, data_type: str, mean: float, standard_deviation: float, source) -> np.ndarray:
    """(type)(mean + nextGaussian() * deviation) per element (TensorRandoms.java:600-629)."""
    if source is None:
        raise TypeError("randomGenerator")
    n = _count(shape, "random tensor creation")
    dt = _dtype(data_type)
    if not math.isfinite(mean):
        raise ValueError(f"random normal mean must be finite: {mean}")
    if not (math.isfinite(standard_deviation) and standard_deviation >= 0.0):
        raise ValueError(f"random normal standard deviation must be finite and non-negative: "
                         f"{standard_deviation}")
    if hasattr(source, "gaussian_block"):
        g = np.asarray(source.gaussian_block(n), np.float64)
    else:
        g = np.array([source.next_gaussian() for _ in range(n)], np.float64)
    return (mean + g * standard_deviation).astype(dt).reshape(tuple(shape))


def uniform(shape, data_type: str, lower_bound_inclusive: float, upper_bound_exclusive: float,
            source) -> np.ndarray:
    """(type) nextDouble(lower, upper) per element (TensorRandoms.java:442-478,783-796)."""
    if source is None:
        raise TypeError("randomGenerator")
    n = _count(shape, "uniform random tensor creation")
    dt = _dtype(data_type)
    if not math.isfinite(lower_bound_inclusive):
        raise ValueError(f"uniform random lower bound must be finite: {lower_bound_inclusive}")
    if not math.isfinite(upper_bound_exclusive):
        raise ValueError(f"uniform random upper bound must be finite: {upper_bound_exclusive}")
    if not lower_bound_inclusive < upper_bound_exclusive:
        raise ValueError("uniform random lower bound must be less than upper bound: "
                         f"lower={lower_bound_inclusive}, upper={upper_bound_exclusive}")
    return _uniform_draws(source, lower_bound_inclusive, upper_bound_exclusive, n,
                          dt).reshape(tuple(shape))


def _fans(weight_shape, data_type, source) -> tuple[float, float]:
    """validateFanInputs (ParameterInitializers.java:375-402): floating type, rank two,
    fanOut = dim 0 and fanIn = dim 1 both positive; returns them as binary64."""
    if source is None:
        raise TypeError("randomGenerator")
    _dtype(data_type)
    shape = tuple(weight_shape)
    if any(d < 0 for d in shape):
        raise ValueError(f"fan-based parameter initialization requires a fully static shape: {shape}")
    if len(shape) != 2:
        raise ValueError(f"fan-based parameter initialization requires rank-two weight shape: {shape}")
    if shape[0] == 0:
        raise ValueError(f"fan-based parameter initialization requires positive outFeatures: {shape[0]}")
    if shape[1] == 0:
        raise ValueError(f"fan-based parameter initialization requires positive inFeatures: {shape[1]}")
    return float(shape[0]), float(shape[1])


def glorot_normal(weight_shape, data_type: str, source) -> np.ndarray:
    fan_out, fan_in = _fans(weight_shape, data_type, source)
    return normal(weight_shape, data_type, 0.0, math.sqrt(2.0 / (fan_in + fan_out)), source)


def glorot_uniform(weight_shape, data_type: str, source) -> np.ndarray:
    fan_out, fan_in = _fans(weight_shape, data_type, source)
    bound = math.sqrt(6.0 / (fan_in + fan_out))
    return uniform(weight_shape, data_type, -bound, bound, source)


def kaiming_relu_normal(weight_shape, data_type: str, source) -> np.ndarray:
    _, fan_in = _fans(weight_shape, data_type, source)
    return normal(weight_shape, data_type, 0.0, math.sqrt(2.0 / fan_in), source)


def kaiming_relu_uniform(weight_shape, data_type: str, source) -> np.ndarray:
    _, fan_in = _fans(weight_shape, data_type, source)
    bound = math.sqrt(6.0 / fan_in)
    return uniform(weight_shape, data_type, -bound, bound, source)


def initialize(shape, data_type: str, policy: ParameterInitialization, source=None) -> np.ndarray:
    """ParameterInitializers.initialize (:100-121): zeros / ones take no source; every other
    policy requires one."""
    if shape is None:
        raise TypeError("shape")
    if data_type is None:
        raise TypeError("dataType")
    if policy is None:
        raise TypeError("initialization")
    if not policy.requires_random_generator:
        if source is not None:
            raise ValueError(f"initialization policy does not accept a random generator: {policy}")
        return zeros(shape, data_type) if policy.kind == "zeros" else ones(shape, data_type)
    if source is None:
        raise ValueError(f"initialization policy requires a random generator: {policy}")
    k = policy.kind
    if k == "normal":
        return normal(shape, data_type, policy.first, policy.second, source)
    if k == "uniform":
        return uniform(shape, data_type, policy.first, policy.second, source)
    return {"glorot_normal": glorot_normal, "glorot_uniform": glorot_uniform,
            "kaiming_relu_normal": kaiming_relu_normal,
            "kaiming_relu_uniform": kaiming_relu_uniform}[k](shape, data_type, source)


def builder_step_seed(seed: int, step: int) -> int:
    """seed + 0x9E3779B97F4A7C15 * step with Java long wraparound (ModelBuilder.java:492-494)."""
    return _java_long(int(seed) + STEP_SEED * int(step))


def builder_parameters(spec, seed: int = 0, data_type: str = "FLOAT32",
                       policy: ParameterInitialization = ParameterInitialization("glorot_uniform")):
    """Weights [out, in] and biases of `Model.builder().seed(seed)` for the Linear chain `spec`
    (an MlpSpec): the steps are appended as linear(out[, bias]) followed by the layer's
    activation step if it has one, so layer k's generator is created from the seed of its own
    step index. Biases are exact zeros (None for a bias-free layer)."""
    Ws, bs = [], []
    step = 0
    for layer in spec.layers:
        source = L64X128MixRandom(builder_step_seed(seed, step))
        Ws.append(initialize((layer.fan_out, layer.fan_in), data_type, policy, source))
        bs.append(zeros((layer.fan_out,), data_type) if layer.bias else None)
        step += 1
        if layer.activation is not None:
            step += 1
    return Ws, bs
