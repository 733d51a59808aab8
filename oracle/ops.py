"""numpy-facing wrappers of the oracle's C loops (TEST INFRASTRUCTURE ONLY).

Every function takes numpy arrays, which may be strided or broadcast views
(np.broadcast_to, transposes, slices): the C loop reads them through their
own strides exactly as Spar's logical_value does (core/tensor.cpp:405-415),
and returns a new contiguous array.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np

from . import fn, lib, ptr, u64

BINARY = {"add": 0, "subtract": 1, "multiply": 2, "divide": 3, "equal": 4, "not_equal": 5,
          "less": 6, "less_equal": 7, "greater": 8, "greater_equal": 9}
UNARY = {"negate": 0, "square": 1, "reciprocal": 2, "exp": 3, "log": 4, "sqrt": 5,
         "sigmoid": 6, "silu": 7, "tanh": 8, "gelu": 9, "gelu_derivative": 10}


def _view(array: np.ndarray):
    """(pointer, rank, extents, element strides, offset) of a numpy view."""
    itemsize = array.itemsize
    for s in array.strides:
        if s < 0 or s % itemsize:
            raise ValueError("oracle views need non-negative element strides")
    extents = u64(array.shape)
    strides = u64([s // itemsize for s in array.strides])
    return ptr(array), array.ndim, extents, strides, 0


def _op(table, op):
    return table[op] if isinstance(op, str) else int(op)


def binary(a: np.ndarray, b: np.ndarray, op) -> np.ndarray:
    """binary_values (ops/elementwise.cpp:33-46) over the broadcast shape."""
    shape = np.broadcast_shapes(a.shape, b.shape)
    a = np.broadcast_to(a, shape)
    b = np.broadcast_to(b, shape)
    out = np.empty(shape, dtype=a.dtype)
    pa, rank, extents, sa, oa = _view(a)
    pb, _, _, sb, ob = _view(b)
    fn("spar_oracle_binary", a.dtype)(ptr(out), pa, sa, oa, pb, sb, ob, rank, extents,
                                      _op(BINARY, op))
    return out


def scalar(a: np.ndarray, op, value: float) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty_like(a)
    fn("spar_oracle_scalar", a.dtype)(ptr(out), ptr(a), a.size, _op(BINARY, op), float(value))
    return out


def unary(a: np.ndarray, op) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty_like(a)
    fn("spar_oracle_unary", a.dtype)(ptr(out), ptr(a), a.size, _op(UNARY, op))
    return out


def full_reduce(a: np.ndarray, kind: str):
    """sum / mean / max over all elements in logical order (reduction.cpp:21-60)."""
    p, rank, extents, strides, offset = _view(a)
    value = fn(f"spar_oracle_{kind}", a.dtype)(p, rank, extents, strides, offset)
    return a.dtype.type(value)


def _mask(ndim: int, axes) -> int:
    mask = 0
    for axis in axes:
        mask |= 1 << axis
    return mask


def axis_sum(a: np.ndarray, axes) -> np.ndarray:
    """axis_sum_values (ops/reduction.cpp:110-145); output has the kept axes."""
    axes = sorted(set(axes))
    kept = [d for i, d in enumerate(a.shape) if i not in axes]
    out = np.empty(kept, dtype=a.dtype)
    p, rank, extents, strides, offset = _view(a)
    fn("spar_oracle_axis_sum", a.dtype)(ptr(out), out.size, p, rank, extents, strides, offset,
                                        _mask(a.ndim, axes))
    return out


def axis_max(a: np.ndarray, axes):
    """Build-defined axis max/argmax: (values, int64 indices) over kept axes."""
    axes = sorted(set(axes))
    kept = [d for i, d in enumerate(a.shape) if i not in axes]
    values = np.empty(kept, dtype=a.dtype)
    indices = np.empty(kept, dtype=np.int64)
    scratch = np.empty(max(values.size, 1), dtype=np.uint8)
    p, rank, extents, strides, offset = _view(a)
    fn("spar_oracle_axis_max", a.dtype)(ptr(values), ptr(indices), values.size, p, rank, extents,
                                        strides, offset, _mask(a.ndim, axes), ptr(scratch))
    return values, indices


def reduce_gradient(gradient: np.ndarray, original_shape) -> np.ndarray:
    """reduce_gradient_values (core/tensor.cpp:572-595)."""
    out = np.empty(tuple(original_shape), dtype=gradient.dtype)
    p, rank, extents, strides, offset = _view(gradient)
    fn("spar_oracle_reduce_gradient", gradient.dtype)(ptr(out), p, rank, extents, strides, offset,
                                                      len(original_shape), u64(original_shape))
    return out


def strided_copy(a: np.ndarray) -> np.ndarray:
    """materialize_cpu_logical (core/tensor.cpp:142-167)."""
    out = np.empty(a.shape, dtype=a.dtype)
    p, rank, extents, strides, offset = _view(a)
    lib().spar_oracle_strided_copy(ptr(out), p, a.itemsize, rank, extents, strides, offset)
    return out


def softmax_axis(a: np.ndarray, axis: int):
    """axis_softmax_values (ops/softmax.cpp:42-108): (probabilities, undefined)."""
    out = np.empty(a.shape, dtype=a.dtype)
    outer = int(np.prod(a.shape[:axis], dtype=np.int64))
    inner = int(np.prod(a.shape[axis + 1:], dtype=np.int64))
    undefined = np.empty(outer * inner, dtype=np.uint8)
    p, rank, extents, strides, offset = _view(a)
    fn("spar_oracle_softmax_axis", a.dtype)(ptr(out), ptr(undefined), p, rank, extents, strides,
                                            offset, axis)
    return out, undefined


def softmax_full(a: np.ndarray) -> np.ndarray:
    """softmax_values (ops/softmax.cpp:190-239); contiguous input."""
    a = np.ascontiguousarray(a)
    out = np.empty_like(a)
    fn("spar_oracle_softmax_full", a.dtype)(ptr(out), ptr(a), a.size)
    return out


def softmax_full_undefined(a: np.ndarray) -> bool:
    a = np.ascontiguousarray(a)
    return bool(fn("spar_oracle_softmax_full_undefined", a.dtype)(ptr(a), a.size))


def log_softmax(a: np.ndarray, axis=None):
    """log_softmax_values (ops/softmax.cpp:342-404): (log probs, undefined)."""
    out = np.empty(a.shape, dtype=a.dtype)
    if axis is None:
        slices = 1
    else:
        slices = int(np.prod(a.shape[:axis], dtype=np.int64)) * int(
            np.prod(a.shape[axis + 1:], dtype=np.int64))
    undefined = np.empty(slices, dtype=np.uint8)
    p, rank, extents, strides, offset = _view(a)
    fn("spar_oracle_log_softmax", a.dtype)(ptr(out), ptr(undefined), p, rank, extents, strides,
                                           offset, -1 if axis is None else axis)
    return out, undefined


def softmax_axis_backward(gradient: np.ndarray, output: np.ndarray, undefined: np.ndarray,
                          axis: int) -> np.ndarray:
    """axis_softmax_gradient (ops/softmax.cpp:110-150)."""
    gradient = np.ascontiguousarray(gradient)
    output = np.ascontiguousarray(output)
    undefined = np.ascontiguousarray(undefined, dtype=np.uint8)
    out = np.empty_like(output)
    fn("spar_oracle_softmax_axis_backward", output.dtype)(
        ptr(out), ptr(gradient), ptr(output), ptr(undefined), output.ndim, u64(output.shape), axis)
    return out


def softmax_full_backward(gradient: np.ndarray, output: np.ndarray, undefined: bool) -> np.ndarray:
    """softmax_gradient (ops/softmax.cpp:167-188)."""
    gradient = np.ascontiguousarray(gradient)
    output = np.ascontiguousarray(output)
    out = np.empty_like(output)
    fn("spar_oracle_softmax_full_backward", output.dtype)(ptr(out), ptr(gradient), ptr(output),
                                                          output.size, int(undefined))
    return out


def log_softmax_backward(gradient: np.ndarray, log_probabilities: np.ndarray,
                         undefined: np.ndarray, axis=None) -> np.ndarray:
    """log_softmax_gradient (ops/softmax.cpp:406-444)."""
    gradient = np.ascontiguousarray(gradient)
    lp = np.ascontiguousarray(log_probabilities)
    undefined = np.ascontiguousarray(undefined, dtype=np.uint8)
    out = np.empty_like(lp)
    if axis is None:
        outer, extent, inner = 1, lp.size, 1
    else:
        outer = int(np.prod(lp.shape[:axis], dtype=np.int64))
        extent = lp.shape[axis]
        inner = int(np.prod(lp.shape[axis + 1:], dtype=np.int64))
    fn("spar_oracle_log_softmax_backward", lp.dtype)(ptr(out), ptr(gradient), ptr(lp),
                                                     ptr(undefined), outer, extent, inner)
    return out


def add_in_place(destination: np.ndarray, source: np.ndarray) -> None:
    fn("spar_oracle_add_in_place", destination.dtype)(ptr(destination), ptr(source),
                                                      destination.size)


class Random:
    """core/random.cpp:12-38 restated over the C loop."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed)

    def next_u64(self) -> int:
        return int(lib().spar_oracle_next_u64(ctypes.byref(self.state)))

    def uniform_float(self) -> float:
        return float(lib().spar_oracle_uniform_float(ctypes.byref(self.state)))

    def uniform_double(self) -> float:
        return float(lib().spar_oracle_uniform_double(ctypes.byref(self.state)))

    def uniform(self, shape, dtype=np.float32, low=0.0, high=1.0) -> np.ndarray:
        """random_uniform (core/random.cpp:40-80)."""
        out = np.empty(shape, dtype=dtype)
        fn("spar_oracle_random_uniform", dtype)(ptr(out), out.size, ctypes.byref(self.state),
                                                float(low), float(high))
        return out

    def normal(self, shape, dtype=np.float32, mean=0.0, stddev=1.0) -> np.ndarray:
        """Build-defined Box-Muller normal sampler on uniform_double draws."""
        out = np.empty(shape, dtype=dtype)
        fn("spar_oracle_random_normal", dtype)(ptr(out), out.size, ctypes.byref(self.state),
                                               float(mean), float(stddev))
        return out


# ------------------------------------------------ optimizer and gradient norm

def adamw_correction(beta: float, step: int) -> float:
    """1 - beta^step (optim/adamw.cpp:48-49), with the C library's pow."""
    return float(lib().spar_oracle_adamw_correction(float(beta), int(step)))


def adamw(parameter: np.ndarray, gradient: np.ndarray, first: np.ndarray, second: np.ndarray,
          learning_rate: float, beta1: float, beta2: float, epsilon: float, weight_decay: float,
          first_correction: float, second_correction: float) -> None:
    """update_values (optim/adamw.cpp:37-61) in place on contiguous arrays."""
    for a in (parameter, gradient, first, second):
        if not a.flags.c_contiguous or a.dtype != parameter.dtype or a.size != parameter.size:
            raise ValueError("adamw takes contiguous arrays of one dtype and size")
    fn("spar_oracle_adamw", parameter.dtype)(
        ptr(parameter), ptr(gradient), ptr(first), ptr(second), parameter.size,
        float(learning_rate), float(beta1), float(beta2), float(epsilon), float(weight_decay),
        float(first_correction), float(second_correction))


class SumSquares:
    """StableSumSquares (training/gradients.cpp:28-88): `add` feeds elements in
    order through the C loop; `combine` and `norm` are the host-side rules."""

    def __init__(self):
        self.state = np.array([0.0, 1.0], np.float64)
        self.flags = np.zeros(2, np.int32)

    @property
    def scale(self) -> float:
        return float(self.state[0])

    @property
    def scaled_sum_squares(self) -> float:
        return float(self.state[1])

    @property
    def has_infinity(self) -> bool:
        return bool(self.flags[0])

    @property
    def has_nan(self) -> bool:
        return bool(self.flags[1])

    def add(self, values: np.ndarray) -> "SumSquares":
        values = np.ascontiguousarray(values)
        fn("spar_oracle_sum_squares_add", values.dtype)(ptr(self.state), ptr(self.flags),
                                                        ptr(values), values.size)
        return self

    def combine(self, scale: float, scaled_sum_squares: float, has_infinity: bool,
                has_nan: bool) -> "SumSquares":
        """gradients.cpp:57-77."""
        self.flags[1] |= int(bool(has_nan))
        self.flags[0] |= int(bool(has_infinity))
        if scale == 0.0:
            return self
        if self.state[0] == 0.0:
            self.state[:] = (scale, scaled_sum_squares)
            return self
        mine, total = self.state[0], self.state[1]
        if mine < scale:
            ratio = mine / scale
            self.state[:] = (scale, scaled_sum_squares + total * ratio * ratio)
        else:
            ratio = scale / mine
            self.state[1] = total + scaled_sum_squares * ratio * ratio
        return self

    def norm(self) -> float:
        """gradients.cpp:79-87."""
        if self.has_nan:
            return math.nan
        if self.has_infinity:
            return math.inf
        scale = float(self.state[0])
        return 0.0 if scale == 0.0 else scale * math.sqrt(float(self.state[1]))


def scale(values: np.ndarray, factor: float) -> None:
    """scale_gradient (training/gradients.cpp:97-101) in place."""
    if not values.flags.c_contiguous:
        raise ValueError("scale takes a contiguous array")
    fn("spar_oracle_scale", values.dtype)(ptr(values), values.size, float(factor))
