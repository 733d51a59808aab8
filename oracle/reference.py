"""Restatement of Spar's CPU tensor, ops and autograd layer (TEST INFRASTRUCTURE ONLY).

`RTensor` mirrors spar::Tensor on the CPU path: a view (shape, element
strides, offset) over a shared 1-D numpy storage, with the reference's
autograd graph.  Arithmetic loops run in the oracle's C restatement
(oracle/spar_oracle.c) so every value is computed in the reference's order
with its float operations; this module restates the host-side logic around
them: view metadata (core/tensor.cpp:237-346), broadcast rules (:549-570),
the backward rules of every op (ops/*.cpp) and the engine
(autograd/autograd.cpp:43-265), including its contribution clones and
in-place accumulation order.  The product (spar_amd/) never imports it.

Its backward rules are pinned against torch.autograd in float64 and central
differences by tests/test_oracle_autograd_cpu.py.
"""
from __future__ import annotations

import math
from typing import Callable, List, Optional

import numpy as np
from numpy.lib.stride_tricks import as_strided

from . import ops as C


class _Meta:
    __slots__ = ("requires_grad", "grad_fn", "leaf_grad")

    def __init__(self):
        self.requires_grad = False
        self.grad_fn: Optional[_Node] = None
        self.leaf_grad: Optional[RTensor] = None


class _Node:
    __slots__ = ("parents", "backward")

    def __init__(self, parents, backward):
        self.parents = parents  # list of (meta, shape, dtype)
        self.backward = backward


def _contiguous_strides(shape):
    strides = [0] * len(shape)
    running = 1
    for axis in range(len(shape) - 1, -1, -1):
        strides[axis] = running
        running *= shape[axis]
    return tuple(strides)


class RTensor:
    """A strided view over shared storage with Spar's autograd metadata."""

    def __init__(self, storage: np.ndarray, shape, strides=None, offset=0):
        self.storage = storage
        self.shape = tuple(int(d) for d in shape)
        self.strides = tuple(strides) if strides is not None else _contiguous_strides(self.shape)
        self.offset = int(offset)
        self.meta = _Meta()

    # ------------------------------------------------------------ factories
    @staticmethod
    def of(array: np.ndarray, requires_grad: bool = False) -> "RTensor":
        array = np.array(array, order="C", copy=True)  # keeps rank 0
        t = RTensor(array.reshape(-1), array.shape)
        if requires_grad:
            t.set_requires_grad(True)
        return t

    @property
    def dtype(self):
        return self.storage.dtype

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    def view(self) -> np.ndarray:
        """numpy view of the logical values (no copy)."""
        item = self.storage.itemsize
        base = self.storage[self.offset:] if self.numel else self.storage[:0]
        return as_strided(base, shape=self.shape, strides=[s * item for s in self.strides],
                          writeable=False)

    def numpy(self) -> np.ndarray:
        return C.strided_copy(self.view()) if self.numel else np.empty(self.shape, self.dtype)

    def is_contiguous(self) -> bool:
        # core/tensor.cpp:113-128
        if self.numel == 0 or not self.shape:
            return True
        expected = 1
        for axis in range(len(self.shape) - 1, -1, -1):
            if self.shape[axis] > 1 and self.strides[axis] != expected:
                return False
            expected *= self.shape[axis]
        return True

    # ------------------------------------------------------------- autograd
    @property
    def requires_grad(self) -> bool:
        return self.meta.requires_grad

    def set_requires_grad(self, enabled=True):
        self.meta.requires_grad = enabled

    def grad(self) -> "RTensor":
        return self.meta.leaf_grad

    def detach(self) -> "RTensor":
        return RTensor(self.storage, self.shape, self.strides, self.offset)

    def clone(self) -> "RTensor":
        out = RTensor(self.numpy().reshape(-1), self.shape)
        if self.requires_grad:
            _record(out, [self], lambda g: [g])
        return out

    def contiguous(self) -> "RTensor":
        if self.is_contiguous():
            return self
        return self.clone()

    def reshape(self, shape) -> "RTensor":
        if not self.is_contiguous():
            raise ValueError("reshape requires a contiguous tensor")
        out = RTensor(self.storage, shape, None, self.offset)
        if self.requires_grad:
            original = self.shape
            _record(out, [self], lambda g: [g.reshape(original)])
        return out

    def transpose(self, a: int, b: int) -> "RTensor":
        shape = list(self.shape)
        strides = list(self.strides)
        shape[a], shape[b] = shape[b], shape[a]
        strides[a], strides[b] = strides[b], strides[a]
        out = RTensor(self.storage, shape, strides, self.offset)
        if self.requires_grad:
            _record(out, [self], lambda g: [g.transpose(a, b).contiguous()])
        return out

    def permute(self, axes) -> "RTensor":
        shape = [self.shape[a] for a in axes]
        strides = [self.strides[a] for a in axes]
        inverse = [0] * len(axes)
        for result_axis, source_axis in enumerate(axes):
            inverse[source_axis] = result_axis
        out = RTensor(self.storage, shape, strides, self.offset)
        if self.requires_grad:
            _record(out, [self], lambda g: [g.permute(inverse).contiguous()])
        return out

    def expand(self, shape) -> "RTensor":
        # core/tensor.cpp:313-342
        shape = tuple(shape)
        leading = len(shape) - len(self.shape)
        strides = [0] * len(shape)
        for axis, extent in enumerate(self.shape):
            target = shape[leading + axis]
            if extent == target:
                strides[leading + axis] = self.strides[axis]
            elif extent != 1:
                raise ValueError("expand dimensions are not broadcast-compatible")
        out = RTensor(self.storage, shape, strides, self.offset)
        if self.requires_grad:
            original = self.shape
            _record(out, [self], lambda g: [reduce_gradient_to_shape(g, original)])
        return out

    def narrow(self, axis: int, start: int, length: int) -> "RTensor":
        """Build-defined view (the reference has no slice op): the backward
        rule places the gradient into zeros of the original shape."""
        shape = list(self.shape)
        shape[axis] = length
        out = RTensor(self.storage, shape, self.strides, self.offset + start * self.strides[axis])
        if self.requires_grad:
            original = self.shape
            dtype = self.dtype

            def backward(g):
                full = np.zeros(original, dtype=dtype)
                index = [slice(None)] * len(original)
                index[axis] = slice(start, start + length)
                full[tuple(index)] = g.numpy()
                return [RTensor.of(full)]

            _record(out, [self], backward)
        return out

    def backward(self):
        _backward(self)


def _record(output: RTensor, parents: List[RTensor], backward: Callable):
    # autograd.cpp:43-68
    output.meta = _Meta()
    output.meta.requires_grad = True
    output.meta.grad_fn = _Node([(p.meta, p.shape, p.dtype) for p in parents], backward)


def _backward(loss: RTensor):
    # autograd.cpp:201-265
    order = []
    visited = set()

    def visit(meta):
        if meta is None or not meta.requires_grad or id(meta) in visited:
            return
        visited.add(id(meta))
        if meta.grad_fn is not None:
            for parent_meta, _, _ in meta.grad_fn.parents:
                visit(parent_meta)
        order.append(meta)

    visit(loss.meta)
    gradients = {id(loss.meta): RTensor.of(np.ones(loss.shape, dtype=loss.dtype))}
    for meta in reversed(order):
        gradient = gradients[id(meta)]
        if meta.grad_fn is None:
            if meta.leaf_grad is not None:
                _add_gradient_values(meta.leaf_grad, gradient)
            else:
                meta.leaf_grad = gradient.clone()
            continue
        contributions = meta.grad_fn.backward(gradient)
        assert len(contributions) == len(meta.grad_fn.parents)
        for contribution, (parent_meta, shape, dtype) in zip(contributions, meta.grad_fn.parents):
            assert contribution.shape == tuple(shape), (contribution.shape, shape)
            independent = contribution.detach().clone()  # autograd.cpp:145
            existing = gradients.get(id(parent_meta))
            if existing is None:
                gradients[id(parent_meta)] = independent
            else:
                _add_gradient_values(existing, independent)


def _add_gradient_values(destination: RTensor, contribution: RTensor):
    # autograd.cpp:114-120: destination[i] += contribution[i]
    assert destination.is_contiguous() and contribution.is_contiguous()
    dst = destination.storage[destination.offset:destination.offset + destination.numel]
    src = np.ascontiguousarray(contribution.numpy()).reshape(-1)
    C.add_in_place(dst, src)


# --------------------------------------------------------------- helpers

def broadcast_shape(left, right):
    # core/tensor.cpp:549-570
    rank = max(len(left), len(right))
    out = [1] * rank
    for offset in range(rank):
        a = left[len(left) - 1 - offset] if offset < len(left) else 1
        b = right[len(right) - 1 - offset] if offset < len(right) else 1
        if a == b:
            out[rank - 1 - offset] = a
        elif a == 1:
            out[rank - 1 - offset] = b
        elif b == 1:
            out[rank - 1 - offset] = a
        else:
            raise ValueError("Tensor shapes are not broadcast-compatible")
    return tuple(out)


def reduce_gradient_to_shape(gradient: RTensor, shape) -> RTensor:
    # core/tensor.cpp:572-595
    return RTensor.of(C.reduce_gradient(gradient.view(), tuple(shape)))


def _fresh(values: np.ndarray) -> RTensor:
    return RTensor.of(values)


# ------------------------------------------------------------ elementwise

def _binary_values(a: RTensor, b: RTensor, op: str) -> RTensor:
    shape = broadcast_shape(a.shape, b.shape)
    return _fresh(C.binary(a.detach().expand(shape).view(), b.detach().expand(shape).view(), op))


def _requiring(a, b):
    return [t for t in (a, b) if t.requires_grad]


def add(a: RTensor, b: RTensor) -> RTensor:
    out = _binary_values(a, b, "add")
    if a.requires_grad or b.requires_grad:
        ga, gb, sa, sb = a.requires_grad, b.requires_grad, a.shape, b.shape
        _record(out, _requiring(a, b), lambda g: ([reduce_gradient_to_shape(g, sa)] if ga else [])
                + ([reduce_gradient_to_shape(g, sb)] if gb else []))
    return out


def subtract(a: RTensor, b: RTensor) -> RTensor:
    out = _binary_values(a, b, "subtract")
    if a.requires_grad or b.requires_grad:
        ga, gb, sa, sb = a.requires_grad, b.requires_grad, a.shape, b.shape

        def backward(g):
            result = []
            if ga:
                result.append(reduce_gradient_to_shape(g, sa))
            if gb:
                result.append(reduce_gradient_to_shape(multiply_scalar(g, -1.0), sb))
            return result

        _record(out, _requiring(a, b), backward)
    return out


def multiply(a: RTensor, b: RTensor) -> RTensor:
    out = _binary_values(a, b, "multiply")
    if a.requires_grad or b.requires_grad:
        ga, gb, sa, sb = a.requires_grad, b.requires_grad, a.shape, b.shape
        saved_a = a.detach().clone() if gb else None  # elementwise.cpp:142-147
        saved_b = b.detach().clone() if ga else None

        def backward(g):
            result = []
            if ga:
                result.append(reduce_gradient_to_shape(multiply(g, saved_b), sa))
            if gb:
                result.append(reduce_gradient_to_shape(multiply(g, saved_a), sb))
            return result

        _record(out, _requiring(a, b), backward)
    return out


def divide(a: RTensor, b: RTensor) -> RTensor:
    out = _binary_values(a, b, "divide")
    if a.requires_grad or b.requires_grad:
        ga, gb, sa, sb = a.requires_grad, b.requires_grad, a.shape, b.shape
        saved_a = a.detach().clone() if gb else None
        saved_b = b.detach().clone()

        def backward(g):
            result = []
            if ga:
                result.append(reduce_gradient_to_shape(divide(g, saved_b), sa))
            if gb:
                denominator = multiply(saved_b, saved_b)
                numerator = multiply(g, saved_a)
                result.append(reduce_gradient_to_shape(
                    multiply_scalar(divide(numerator, denominator), -1.0), sb))
            return result

        _record(out, _requiring(a, b), backward)
    return out


def compare(a: RTensor, b: RTensor, op: str) -> RTensor:
    return _binary_values(a, b, op)


# ----------------------------------------------------------------- scalar

def _scalar(x: RTensor, op: str, value: float) -> RTensor:
    if not x.is_contiguous():
        raise ValueError("Scalar operations currently require contiguous tensors")
    return _fresh(C.scalar(x.numpy(), op, value))


def add_scalar(x, value):
    out = _scalar(x, "add", value)
    if x.requires_grad:
        _record(out, [x], lambda g: [g])
    return out


def subtract_scalar(x, value):
    out = _scalar(x, "subtract", value)
    if x.requires_grad:
        _record(out, [x], lambda g: [g])
    return out


def multiply_scalar(x, value):
    out = _scalar(x, "multiply", value)
    if x.requires_grad:
        _record(out, [x], lambda g: [multiply_scalar(g, value)])
    return out


def divide_scalar(x, value):
    out = _scalar(x, "divide", value)
    if x.requires_grad:
        _record(out, [x], lambda g: [divide_scalar(g, value)])
    return out


# ------------------------------------------------------------------ unary

def _unary(x: RTensor, op: str) -> RTensor:
    if not x.is_contiguous():
        raise ValueError("Unary operations currently require contiguous tensors")
    return _fresh(C.unary(x.numpy(), op))


def negate(x):
    out = _unary(x, "negate")
    if x.requires_grad:
        _record(out, [x], lambda g: [multiply_scalar(g, -1.0)])
    return out


def square(x):
    out = _unary(x, "square")
    if x.requires_grad:
        saved = x.detach().clone()
        _record(out, [x], lambda g: [multiply(g, multiply_scalar(saved, 2.0))])
    return out


def reciprocal(x):
    out = _unary(x, "reciprocal")
    if x.requires_grad:
        saved = x.detach().clone()
        _record(out, [x], lambda g: [multiply_scalar(divide(g, multiply(saved, saved)), -1.0)])
    return out


def exp(x):
    out = _unary(x, "exp")
    if x.requires_grad:
        saved = out.detach().clone()
        _record(out, [x], lambda g: [multiply(g, saved)])
    return out


def log(x):
    out = _unary(x, "log")
    if x.requires_grad:
        saved = x.detach().clone()
        _record(out, [x], lambda g: [divide(g, saved)])
    return out


def sqrt(x):
    out = _unary(x, "sqrt")
    if x.requires_grad:
        saved = out.detach().clone()
        _record(out, [x], lambda g: [divide(g, multiply_scalar(saved, 2.0))])
    return out


def sigmoid(x):
    out = _unary(x, "sigmoid")
    if x.requires_grad:
        saved = out.detach().clone()
        _record(out, [x], lambda g: [multiply(g, multiply(saved, add_scalar(
            multiply_scalar(saved, -1.0), 1.0)))])
    return out


def silu(x):
    out = _unary(x, "silu")
    if x.requires_grad:
        saved = x.detach().clone()

        def backward(g):
            s = sigmoid(saved)
            one_minus = add_scalar(multiply_scalar(s, -1.0), 1.0)
            slope = multiply(s, one_minus)
            return [multiply(g, add(s, multiply(saved, slope)))]

        _record(out, [x], backward)
    return out


def tanh(x):
    """Build-defined backward: g * (1 - y*y) composed from ops."""
    out = _unary(x, "tanh")
    if x.requires_grad:
        saved = out.detach().clone()
        _record(out, [x], lambda g: [multiply(g, add_scalar(
            multiply_scalar(multiply(saved, saved), -1.0), 1.0))])
    return out


def gelu(x):
    """Build-defined backward: g * gelu'(x), gelu' evaluated in double."""
    out = _unary(x, "gelu")
    if x.requires_grad:
        saved = x.detach().clone()
        _record(out, [x], lambda g: [multiply(g, _unary(saved, "gelu_derivative"))])
    return out


# ------------------------------------------------------------- reductions

def _fill(shape, value, dtype) -> RTensor:
    return RTensor.of(np.full(shape, value, dtype=dtype))


def sum(x: RTensor, axes=None, keepdim=False) -> RTensor:
    if axes is None:
        out = RTensor.of(np.array(C.full_reduce(x.view(), "sum"), dtype=x.dtype))
        if x.requires_grad:
            shape, dtype = x.shape, x.dtype
            # reduction.cpp:200-212: fill with gradient[0]
            _record(out, [x], lambda g: [_fill(shape, g.numpy().reshape(-1)[0], dtype)])
        return out
    axes = sorted(set([axes] if isinstance(axes, int) else axes))
    values = C.axis_sum(x.view(), axes)
    out_shape = _reduced_shape(x.shape, axes, keepdim)
    out = RTensor.of(values.reshape(out_shape))
    if x.requires_grad:
        shape = x.shape
        _record(out, [x], lambda g: [_restore_and_expand(g, shape, axes, keepdim)])
    return out


def mean(x: RTensor, axes=None, keepdim=False) -> RTensor:
    if axes is None:
        out = RTensor.of(np.array(C.full_reduce(x.view(), "mean"), dtype=x.dtype))
        if x.requires_grad:
            shape, dtype, n = x.shape, x.dtype, x.numel
            # reduction.cpp:263-277: g / (T)n
            _record(out, [x], lambda g: [_fill(
                shape, C.scalar(g.numpy().reshape(1), "divide", float(n))[0], dtype)])
        return out
    axes = sorted(set([axes] if isinstance(axes, int) else axes))
    count = int(np.prod([x.shape[a] for a in axes]))
    summed = C.axis_sum(x.view(), axes)
    values = C.scalar(summed, "divide", float(count))  # reduction.cpp:294-298
    out = RTensor.of(values.reshape(_reduced_shape(x.shape, axes, keepdim)))
    if x.requires_grad:
        shape = x.shape
        _record(out, [x], lambda g: [divide_scalar(
            _restore_and_expand(g, shape, axes, keepdim), float(count))])
    return out


def _reduced_shape(shape, axes, keepdim):
    out = []
    for axis, extent in enumerate(shape):
        if axis in axes:
            if keepdim:
                out.append(1)
        else:
            out.append(extent)
    return tuple(out)


def _restore_and_expand(g: RTensor, shape, axes, keepdim):
    # reduction.cpp:147-165
    restored = g
    if not keepdim:
        dims = [1] * len(shape)
        gi = 0
        for axis in range(len(shape)):
            if axis not in axes:
                dims[axis] = g.shape[gi]
                gi += 1
        restored = g.reshape(dims)
    return restored.expand(shape).contiguous()


# ---------------------------------------------------------------- softmax

def softmax(x: RTensor, axis=None) -> RTensor:
    if axis is None:
        values = C.softmax_full(x.numpy())
        undefined = C.softmax_full_undefined(x.numpy())
        out = RTensor.of(values)
        if x.requires_grad:
            saved = out.detach().clone()
            _record(out, [x], lambda g: [RTensor.of(
                C.softmax_full_backward(g.numpy(), saved.numpy(), undefined))])
        return out
    values, undefined = C.softmax_axis(x.view(), axis)
    out = RTensor.of(values)
    if x.requires_grad:
        saved = out.detach().clone()
        _record(out, [x], lambda g: [RTensor.of(
            C.softmax_axis_backward(g.numpy(), saved.numpy(), undefined, axis))])
    return out


def log_softmax(x: RTensor, axis=None) -> RTensor:
    values, undefined = C.log_softmax(x.view(), axis)
    out = RTensor.of(values)
    if x.requires_grad:
        saved = out.detach().clone()
        _record(out, [x], lambda g: [RTensor.of(
            C.log_softmax_backward(g.numpy(), saved.numpy(), undefined, axis))])
    return out


# ------------------------------------------------------- normalisation

def rms_norm(x: RTensor, weight: RTensor, epsilon: float = 1.0e-5) -> RTensor:
    """RMSNorm::forward (nn/rmsnorm.cpp:41-53): the reference composes it from
    ops, so autograd runs through each of them."""
    axis = len(x.shape) - 1
    mean_square = mean(square(x), [axis], True)
    denominator = sqrt(add_scalar(mean_square, epsilon))
    return multiply(divide(x, denominator), weight)


def layer_norm(x: RTensor, weight: RTensor, bias: RTensor, epsilon: float = 1.0e-5) -> RTensor:
    """Build-defined LayerNorm as the same composition with centring and a
    bias: (x - mean) / sqrt(mean((x - mean)^2) + eps) * weight + bias."""
    axis = len(x.shape) - 1
    centred = subtract(x, mean(x, [axis], True))
    denominator = sqrt(add_scalar(mean(square(centred), [axis], True), epsilon))
    return add(multiply(divide(centred, denominator), weight), bias)


# ------------------------------------------------------------ cross entropy

def _validated_targets(targets: np.ndarray, classes: int) -> np.ndarray:
    """validated_targets (loss/cross_entropy.cpp:17-46): Int32/Int64 class
    indices in [0, classes), flattened in logical order."""
    if targets.dtype not in (np.int32, np.int64):
        raise ValueError("cross_entropy targets must have Int32 or Int64 dtype")
    flat = np.ascontiguousarray(targets).reshape(-1).astype(np.int64)
    if np.any(flat < 0) or np.any(flat >= classes):
        raise IndexError("cross_entropy target is outside the class range")
    return flat


def _select_nll(lp: RTensor, targets: np.ndarray, rows: np.ndarray, output_shape) -> RTensor:
    """select_nll / nll_values / nll_gradient (loss/cross_entropy.cpp:56-105):
    losses = -lp[row, target]; the gradient is a zero tensor with
    0 - upstream at each (row, target)."""
    classes = lp.shape[-1]
    index = rows * classes + targets
    values = -np.ascontiguousarray(lp.numpy()).reshape(-1)[index]
    out = RTensor.of(values.reshape(tuple(output_shape)))
    if lp.requires_grad:
        shape, dtype = tuple(lp.shape), lp.numpy().dtype

        def backward(g):
            contribution = np.zeros(int(np.prod(shape)), dtype=dtype)
            contribution[index] = contribution[index] - np.ascontiguousarray(g.numpy()).reshape(-1)
            return [RTensor.of(contribution.reshape(shape))]

        _record(out, [lp], backward)
    return out


def _reduce_loss(losses: RTensor, reduction: str) -> RTensor:
    """reduce_loss (loss/cross_entropy.cpp:107-117)."""
    if reduction == "none":
        return losses
    if reduction == "sum":
        return sum(losses)
    if reduction == "mean":
        return mean(losses)
    raise ValueError("cross_entropy received an unknown Reduction")


def cross_entropy(logits: RTensor, targets: np.ndarray, reduction: str = "mean") -> RTensor:
    """cross_entropy, CPU path (loss/cross_entropy.cpp:131-160)."""
    if targets.size == 0:
        raise ValueError("cross_entropy requires at least one target")
    if tuple(targets.shape) != tuple(logits.shape[:-1]):
        raise ValueError("cross_entropy target shape does not match logits")
    classes = logits.shape[-1]
    flat = _validated_targets(targets, classes)
    lp = log_softmax(logits, len(logits.shape) - 1)
    return _reduce_loss(_select_nll(lp, flat, np.arange(flat.size, dtype=np.int64),
                                    targets.shape), reduction)


def language_model_cross_entropy(logits: RTensor, token_ids: np.ndarray,
                                 reduction: str = "mean") -> RTensor:
    """language_model_cross_entropy, CPU path (loss/cross_entropy.cpp:162-212):
    position t of each sequence predicts token t + 1."""
    batch, sequence, classes = logits.shape
    tokens = _validated_targets(token_ids, classes).reshape(batch, sequence)
    targets = tokens[:, 1:].reshape(-1)
    rows = (np.arange(batch, dtype=np.int64)[:, None] * sequence +
            np.arange(sequence - 1, dtype=np.int64)[None, :]).reshape(-1)
    lp = log_softmax(logits, 2)
    return _reduce_loss(_select_nll(lp, targets, rows, (batch, sequence - 1)), reduction)


# ------------------------------------------------ optimizer and gradient norm
#
# Parameters are given by their gradient arrays (None for a Parameter without
# a gradient) and value arrays; the logic below is the CPU path of
# training/gradients.cpp and optim/adamw.cpp on them.

def global_grad_norm(gradients) -> float:
    """global_grad_norm, CPU path (training/gradients.cpp:105-137): one
    StableSumSquares fed every element of every active gradient in order."""
    accumulator = C.SumSquares()
    for gradient in gradients:
        if gradient is not None:
            accumulator.add(gradient)
    return accumulator.norm()


def scale_gradients(gradients, factor: float) -> None:
    """scale_gradients, CPU path (training/gradients.cpp:139-174), in place."""
    if not math.isfinite(factor):
        raise ValueError("Gradient scale factor must be finite")
    for gradient in gradients:
        if gradient is not None:
            C.scale(gradient, factor)


def clip_grad_norm(gradients, max_norm: float):
    """clip_grad_norm (training/gradients.cpp:176-190): (total_norm, scale,
    clipped), scaling the gradients in place when clipped."""
    if not math.isfinite(max_norm) or max_norm < 0.0:
        raise ValueError("Maximum gradient norm must be finite and nonnegative")
    total = global_grad_norm(gradients)
    if not math.isfinite(total):
        raise RuntimeError("Cannot clip nonfinite gradients")
    if total == 0.0 or total <= max_norm:
        return total, 1.0, False
    factor = max_norm / total
    scale_gradients(gradients, factor)
    return total, factor, True


class AdamW:
    """AdamW, CPU path (optim/adamw.cpp:67-170): per-parameter moments (zeros
    of the parameter's dtype on first use) and step counters; `step` updates
    each parameter array with a gradient in place."""

    def __init__(self, parameters, learning_rate=1.0e-3, beta1=0.9, beta2=0.999,
                 epsilon=1.0e-8, weight_decay=0.01):
        self.parameters = list(parameters)
        self.learning_rate = learning_rate
        self.beta1, self.beta2 = beta1, beta2
        self.epsilon, self.weight_decay = epsilon, weight_decay
        self.states = [None] * len(self.parameters)

    def step(self, gradients) -> None:
        for index, (value, gradient) in enumerate(zip(self.parameters, gradients)):
            if gradient is None:
                continue
            if self.states[index] is None:
                self.states[index] = [np.zeros_like(value), np.zeros_like(value), 0]
            state = self.states[index]
            state[2] += 1
            C.adamw(value, np.ascontiguousarray(gradient, value.dtype), state[0], state[1],
                    self.learning_rate, self.beta1, self.beta2, self.epsilon, self.weight_decay,
                    C.adamw_correction(self.beta1, state[2]),
                    C.adamw_correction(self.beta2, state[2]))
