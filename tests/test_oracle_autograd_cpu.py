"""Pins the backward rules of the oracle's autograd restatement
(oracle/reference.py) against an independent implementation.

Every backward-bearing function of the restatement is run in float64 on
seeded inputs and compared with torch.autograd on the same float64 inputs,
and the build-defined rules (gelu, tanh, narrow, the norm compositions) also
with central differences.  torch computes the same derivatives through its
own kernels and graph, so a slip shared by the restatement and the C++
engine it checks (both follow the reference's text) shows up here.  The
loss of every case is sum(f(inputs) * W) with a seeded W, so every gradient
element is exercised with a different weight.

Rules restated, by reference file: elementwise.cpp:72-215 (add, subtract,
multiply, divide with broadcast), scalar.cpp:63-103, unary.cpp:69-160,
reduction.cpp:200-212 and :263-298 (sum/mean), softmax.cpp:110-150,
:253-333, :406-444 and :475-506, tensor.cpp:219-341 (view gradients),
rmsnorm.cpp:50-52, cross_entropy.cpp:56-212 and autograd.cpp:43-265 (the
engine's accumulation).

Mutation checks plant a mistake in the oracle (a flipped sign in divide's
right-hand gradient, a dropped dot term in softmax's backward) and assert
that the comparison fails.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle.reference as R  # noqa: E402
from oracle import ops as O  # noqa: E402

F64 = np.float64
RTOL = 1e-11  # float64 restatement vs torch: different operation order only


def rng(seed):
    return np.random.default_rng(seed)


def normal(seed, shape):
    return rng(seed).standard_normal(shape)


def uniform(seed, shape, low, high):
    return rng(seed).uniform(low, high, shape)


def run_oracle(fn, arrays, weight):
    leaves = [R.RTensor.of(a.astype(F64), requires_grad=True) for a in arrays]
    out = fn(*leaves)
    loss = R.sum(R.multiply(out, R.RTensor.of(weight))) if weight is not None else out
    loss.backward()
    return float(loss.numpy()), [leaf.grad().numpy() if leaf.grad() is not None else None
                                 for leaf in leaves]


def run_torch(fn, arrays, weight):
    leaves = [torch.tensor(a.astype(F64), requires_grad=True) for a in arrays]
    out = fn(*leaves)
    loss = (out * torch.tensor(weight)).sum() if weight is not None else out
    loss.backward()
    return float(loss.detach()), [leaf.grad.numpy() if leaf.grad is not None else None
                                  for leaf in leaves]


def check(oracle_fn, torch_fn, arrays, out_shape=None, seed=99, rtol=RTOL):
    """Compares the oracle's loss and every leaf gradient with torch's."""
    weight = None
    if out_shape is not None:
        weight = normal(seed, out_shape)
    loss_r, grads_r = run_oracle(oracle_fn, arrays, weight)
    loss_t, grads_t = run_torch(torch_fn, arrays, weight)
    assert abs(loss_r - loss_t) <= rtol * max(1.0, abs(loss_t)) * 10, (loss_r, loss_t)
    for k, (gr, gt) in enumerate(zip(grads_r, grads_t)):
        assert gt is not None and gr is not None, f"leaf {k}: gradient missing"
        assert gr.shape == gt.shape, f"leaf {k}: shape {gr.shape} != {gt.shape}"
        scale = max(1.0, float(np.max(np.abs(gt))) if gt.size else 1.0)
        err = float(np.max(np.abs(gr - gt))) if gt.size else 0.0
        assert err <= rtol * scale, f"leaf {k}: max |oracle - torch| = {err:.3e} (scale {scale:.3e})"


# ------------------------------------------------------------- elementwise

BROADCAST_SHAPES = [((3, 1, 5), (4, 5)), ((2, 3, 4), (2, 3, 4)), ((6,), (2, 3, 6)),
                    ((2, 1, 4), (1, 3, 1))]


@pytest.mark.parametrize("sa,sb", BROADCAST_SHAPES)
@pytest.mark.parametrize("op", ["add", "subtract", "multiply", "divide"])
def test_binary_backward_with_broadcast(op, sa, sb):
    a = normal(1, sa)
    b = normal(2, sb) if op != "divide" else uniform(2, sb, 0.5, 2.0) * np.where(
        rng(3).random(sb) < 0.5, -1.0, 1.0)
    shape = np.broadcast_shapes(sa, sb)
    torch_op = {"add": torch.add, "subtract": torch.sub, "multiply": torch.mul,
                "divide": torch.div}[op]
    check(lambda x, y: getattr(R, op)(x, y), torch_op, [a, b], shape)


def test_binary_backward_one_side_requires_grad():
    a, b = normal(4, (3, 4)), uniform(5, (4,), 0.5, 2.0)
    weight = normal(6, (3, 4))
    ta = R.RTensor.of(a, requires_grad=True)
    tb = R.RTensor.of(b)  # no gradient
    R.sum(R.multiply(R.divide(ta, tb), R.RTensor.of(weight))).backward()
    xa = torch.tensor(a, requires_grad=True)
    ((xa / torch.tensor(b)) * torch.tensor(weight)).sum().backward()
    np.testing.assert_allclose(ta.grad().numpy(), xa.grad.numpy(), rtol=0, atol=1e-14)


def test_same_tensor_on_both_sides():
    # x*x and x/x: both parents are the same leaf; the engine accumulates
    a = uniform(7, (5, 3), 0.5, 1.5)
    check(lambda x: R.add(R.multiply(x, x), R.divide(x, R.add(x, x))),
          lambda x: x * x + x / (x + x), [a], (5, 3))


# ------------------------------------------------------------------ scalar

@pytest.mark.parametrize("op,value", [("add_scalar", 1.25), ("subtract_scalar", -3.5),
                                      ("multiply_scalar", -2.5), ("divide_scalar", 3.0)])
def test_scalar_backward(op, value):
    a = normal(8, (4, 6))
    torch_fn = {"add_scalar": lambda x: x + value, "subtract_scalar": lambda x: x - value,
                "multiply_scalar": lambda x: x * value, "divide_scalar": lambda x: x / value}[op]
    check(lambda x: getattr(R, op)(x, value), torch_fn, [a], (4, 6))


# ------------------------------------------------------------------- unary

UNARY = {
    "negate": (lambda x: -x, (-3, 3)),
    "square": (lambda x: x * x, (-3, 3)),
    "reciprocal": (lambda x: 1.0 / x, (0.4, 3)),
    "exp": (torch.exp, (-3, 3)),
    "log": (torch.log, (0.1, 5)),
    "sqrt": (torch.sqrt, (0.1, 5)),
    "sigmoid": (torch.sigmoid, (-6, 6)),
    "silu": (torch.nn.functional.silu, (-6, 6)),
    "tanh": (torch.tanh, (-4, 4)),
    "gelu": (lambda x: torch.nn.functional.gelu(x, approximate="none"), (-5, 5)),
}


@pytest.mark.parametrize("op", sorted(UNARY))
def test_unary_backward(op):
    torch_fn, (low, high) = UNARY[op]
    a = uniform(9, (7, 9), low, high)
    if op == "reciprocal":
        a *= np.where(rng(10).random(a.shape) < 0.5, -1.0, 1.0)
    check(lambda x: getattr(R, op)(x), torch_fn, [a], (7, 9))


def central_difference(f, x, h=1e-6):
    """d/dx_i of f (scalar-valued) by central differences, per element."""
    grad = np.empty_like(x)
    flat = x.reshape(-1)
    out = grad.reshape(-1)
    for i in range(flat.size):
        keep = flat[i]
        flat[i] = keep + h
        up = f(x)
        flat[i] = keep - h
        down = f(x)
        flat[i] = keep
        out[i] = (up - down) / (2 * h)
    return grad


@pytest.mark.parametrize("op", ["gelu", "tanh"])
def test_build_defined_unary_against_central_differences(op):
    a = uniform(11, (3, 5), -4, 4)
    weight = normal(12, (3, 5))
    _, grads = run_oracle(lambda x: getattr(R, op)(x), [a], weight)
    f = (lambda v: float(np.sum(weight * O.unary(v, op))))
    want = central_difference(f, a.copy())
    np.testing.assert_allclose(grads[0], want, rtol=1e-6, atol=1e-8)


# -------------------------------------------------------------- reductions

REDUCE_CASES = [(None, False), ([1], False), ([1], True), ([0, 2], False), ([0, 2], True),
                ([2], True), ([0, 1, 2], False)]


@pytest.mark.parametrize("axes,keepdim", REDUCE_CASES)
@pytest.mark.parametrize("kind", ["sum", "mean"])
def test_reduction_backward(kind, axes, keepdim):
    a = normal(13, (3, 4, 5))

    def torch_fn(x):
        if axes is None:
            return getattr(torch, kind)(x)
        return getattr(torch, kind)(x, dim=axes, keepdim=keepdim)

    out_shape = tuple(np.asarray(torch_fn(torch.tensor(a))).shape)
    check(lambda x: getattr(R, kind)(x, axes, keepdim), torch_fn, [a], out_shape)


def test_reduction_of_view_backward():
    # mean over axis 1 of a transposed view: the gradient lands in the base
    a = normal(14, (6, 4))
    check(lambda x: R.mean(x.transpose(0, 1), [1], True), lambda x: x.t().mean(1, keepdim=True),
          [a], (4, 1))


# ---------------------------------------------------------------- softmax

@pytest.mark.parametrize("axis", [None, 0, 1, 2])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_backward(axis, log):
    a = normal(15, (3, 4, 5)) * 2.0

    def torch_fn(x):
        if axis is None:
            flat = x.reshape(-1)
            y = torch.log_softmax(flat, 0) if log else torch.softmax(flat, 0)
            return y.reshape(x.shape)
        return torch.log_softmax(x, axis) if log else torch.softmax(x, axis)

    fn = R.log_softmax if log else R.softmax
    check(lambda x: fn(x, axis), torch_fn, [a], (3, 4, 5))


def test_softmax_of_transposed_view_backward():
    a = normal(16, (5, 7))
    check(lambda x: R.softmax(x.transpose(0, 1), 1), lambda x: torch.softmax(x.t(), 1), [a], (7, 5))


# ------------------------------------------------------------------ views

VIEW_CASES = {
    "transpose": (lambda x: x.transpose(0, 2), lambda x: x.permute(2, 1, 0), (5, 4, 3)),
    "permute": (lambda x: x.permute([1, 2, 0]), lambda x: x.permute(1, 2, 0), (4, 5, 3)),
    "expand": (lambda x: x.narrow(1, 0, 1).contiguous().expand([2, 3, 3, 5]),
               lambda x: x[:, 0:1].expand(2, 3, 3, 5), (2, 3, 3, 5)),
    "narrow": (lambda x: x.narrow(1, 1, 2).narrow(2, 2, 3), lambda x: x[:, 1:3, 2:5], (3, 2, 3)),
    "reshape": (lambda x: x.reshape([12, 5]), lambda x: x.reshape(12, 5), (12, 5)),
    "contiguous of transpose": (lambda x: x.transpose(0, 1).contiguous(),
                                lambda x: x.transpose(0, 1).contiguous(), (4, 3, 5)),
    "clone": (lambda x: x.clone(), lambda x: x.clone(), (3, 4, 5)),
}


@pytest.mark.parametrize("name", sorted(VIEW_CASES))
def test_view_backward(name):
    oracle_fn, torch_fn, out_shape = VIEW_CASES[name]
    a = normal(17, (3, 4, 5))
    check(oracle_fn, torch_fn, [a], out_shape)


def test_expand_of_broadcast_operand_backward():
    bias = normal(18, (5,))
    check(lambda b: b.expand([3, 4, 5]), lambda b: b.expand(3, 4, 5), [bias], (3, 4, 5))


def test_narrow_against_central_differences():
    a = normal(19, (4, 6))
    weight = normal(20, (2, 3))
    _, grads = run_oracle(lambda x: x.narrow(0, 1, 2).narrow(1, 3, 3), [a], weight)
    want = np.zeros_like(a)
    want[1:3, 3:6] = weight
    np.testing.assert_array_equal(grads[0], want)


# ---------------------------------------------------------- norm compositions

def test_layer_norm_composition_backward():
    x, w, b = normal(21, (6, 8)), uniform(22, (8,), 0.5, 1.5), uniform(23, (8,), -0.1, 0.1)

    def torch_fn(x, w, b):
        mu = x.mean(-1, keepdim=True)
        xc = x - mu
        var = (xc * xc).mean(-1, keepdim=True)
        return xc / torch.sqrt(var + 1e-5) * w + b

    check(lambda x, w, b: R.layer_norm(x, w, b, 1e-5), torch_fn, [x, w, b], (6, 8))
    # and the library form of the same function
    check(lambda x, w, b: R.layer_norm(x, w, b, 1e-5),
          lambda x, w, b: torch.nn.functional.layer_norm(x, (8,), w, b, 1e-5), [x, w, b], (6, 8),
          rtol=1e-9)


def test_layer_norm_on_views_backward():
    base = normal(24, (8, 6))
    w, b = uniform(25, (8,), 0.5, 1.5), uniform(26, (8,), -0.1, 0.1)
    check(lambda x, w, b: R.layer_norm(x.transpose(0, 1), w, b, 1e-5),
          lambda x, w, b: torch.nn.functional.layer_norm(x.t(), (8,), w, b, 1e-5),
          [base, w, b], (6, 8), rtol=1e-9)
    big = normal(27, (9, 12))
    check(lambda x, w, b: R.layer_norm(x.narrow(0, 2, 6).narrow(1, 3, 8), w, b, 1e-5),
          lambda x, w, b: torch.nn.functional.layer_norm(x[2:8, 3:11], (8,), w, b, 1e-5),
          [big, w, b], (6, 8), rtol=1e-9)


def test_rms_norm_composition_backward():
    x, w = normal(28, (5, 16)), uniform(29, (16,), 0.5, 1.5)
    check(lambda x, w: R.rms_norm(x, w, 1e-5),
          lambda x, w: x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-5) * w, [x, w], (5, 16))


def test_layer_norm_against_central_differences():
    x = normal(30, (2, 6))
    w, b = uniform(31, (6,), 0.5, 1.5), uniform(32, (6,), -0.1, 0.1)
    weight = normal(33, (2, 6))
    _, grads = run_oracle(lambda x: R.layer_norm(x, R.RTensor.of(w), R.RTensor.of(b), 1e-5), [x],
                          weight)

    def f(v):
        mu = v.mean(-1, keepdims=True)
        xc = v - mu
        y = xc / np.sqrt((xc * xc).mean(-1, keepdims=True) + 1e-5) * w + b
        return float(np.sum(y * weight))

    np.testing.assert_allclose(grads[0], central_difference(f, x.copy()), rtol=1e-6, atol=1e-8)


# ------------------------------------------------------------- cross entropy

@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_cross_entropy_backward(reduction):
    logits = normal(34, (6, 9)) * 2
    targets = rng(35).integers(0, 9, 6)
    weight_shape = (6,) if reduction == "none" else None

    def oracle_fn(x):
        return R.cross_entropy(x, targets.astype(np.int64), reduction)

    def torch_fn(x):
        return torch.nn.functional.cross_entropy(x, torch.tensor(targets), reduction=reduction)

    check(oracle_fn, torch_fn, [logits], weight_shape)


@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_language_model_cross_entropy_backward(reduction):
    batch, sequence, classes = 2, 5, 7
    logits = normal(36, (batch, sequence, classes))
    tokens = rng(37).integers(0, classes, (batch, sequence))
    weight_shape = (batch, sequence - 1) if reduction == "none" else None

    def torch_fn(x):
        loss = torch.nn.functional.cross_entropy(
            x[:, :-1].reshape(-1, classes), torch.tensor(tokens[:, 1:]).reshape(-1),
            reduction=reduction)
        return loss.reshape(batch, sequence - 1) if reduction == "none" else loss

    check(lambda x: R.language_model_cross_entropy(x, tokens.astype(np.int64), reduction),
          torch_fn, [logits], weight_shape)


# ----------------------------------------------------------------- engine

def test_engine_diamond_and_reuse():
    # x feeds three paths that meet again; w is used twice
    x, w = normal(38, (4, 5)), uniform(39, (5,), 0.5, 1.5)

    def oracle_fn(x, w):
        h = R.multiply(x, w)
        return R.add(R.add(R.exp(R.multiply_scalar(h, 0.1)), R.square(h)),
                     R.multiply(R.softmax(h, 1), w))

    def torch_fn(x, w):
        h = x * w
        return torch.exp(h * 0.1) + h * h + torch.softmax(h, 1) * w

    check(oracle_fn, torch_fn, [x, w], (4, 5))


def test_leaf_gradient_accumulates_across_backward_calls():
    a = normal(40, (3, 4))
    weight = normal(41, (3, 4))
    t = R.RTensor.of(a, requires_grad=True)
    for _ in range(2):
        R.sum(R.multiply(R.tanh(t), R.RTensor.of(weight))).backward()
    x = torch.tensor(a, requires_grad=True)
    for _ in range(2):
        (torch.tanh(x) * torch.tensor(weight)).sum().backward()
    np.testing.assert_allclose(t.grad().numpy(), x.grad.numpy(), rtol=0, atol=1e-14)


def test_engine_float32_matches_float64_rules():
    # the float32 restatement runs the same rules: compare with torch in
    # float32 at float32 tolerance on a broadcast chain
    x, s, b = normal(42, (2, 3, 8)), uniform(43, (2, 1, 8), 0.5, 1.5), uniform(44, (8,), -0.1, 0.1)
    weight = normal(45, (2, 3, 8)).astype(np.float32)
    leaves = [R.RTensor.of(v.astype(np.float32), requires_grad=True) for v in (x, s, b)]
    y = R.softmax(R.add(R.multiply(leaves[0], leaves[1]), leaves[2]), 2)
    R.sum(R.multiply(y, R.RTensor.of(weight))).backward()
    tl = [torch.tensor(v.astype(np.float32), requires_grad=True) for v in (x, s, b)]
    (torch.softmax(tl[0] * tl[1] + tl[2], 2) * torch.tensor(weight)).sum().backward()
    for k in range(3):
        np.testing.assert_allclose(leaves[k].grad().numpy(), tl[k].grad.numpy(), rtol=1e-5,
                                   atol=1e-6)


# -------------------------------------------------------------- mutations

def test_mutation_flipped_divide_sign_is_caught(monkeypatch):
    a, b = normal(46, (3, 4)), uniform(47, (4,), 0.5, 2.0)
    check(R.divide, torch.div, [a, b], (3, 4))  # the rule as written passes
    real = R.multiply_scalar

    def flipped(x, value):
        # divide's right-hand gradient is multiply_scalar(g*a/(b*b), -1.0)
        return real(x, -value if value == -1.0 else value)

    monkeypatch.setattr(R, "multiply_scalar", flipped)
    with pytest.raises(AssertionError):
        check(R.divide, torch.div, [a, b], (3, 4))


def test_mutation_dropped_softmax_dot_term_is_caught(monkeypatch):
    a = normal(48, (4, 6))
    check(lambda x: R.softmax(x, 1), lambda x: torch.softmax(x, 1), [a], (4, 6))

    def no_dot(gradient, output, undefined, axis):
        return gradient * output  # y * g without the - y * sum(g * y) term

    monkeypatch.setattr(R.C, "softmax_axis_backward", no_dot)
    with pytest.raises(AssertionError):
        check(lambda x: R.softmax(x, 1), lambda x: torch.softmax(x, 1), [a], (4, 6))


def test_mutation_wrong_broadcast_reduction_is_caught(monkeypatch):
    a, bias = normal(49, (3, 5)), normal(50, (5,))
    check(R.add, torch.add, [a, bias], (3, 5))

    def first_row_only(gradient, shape):
        values = gradient.numpy()
        return R.RTensor.of(values.reshape(-1, *shape)[0].copy() if values.shape != tuple(shape)
                            else values)

    monkeypatch.setattr(R, "reduce_gradient_to_shape", first_row_only)
    with pytest.raises(AssertionError):
        check(R.add, torch.add, [a, bias], (3, 5))
