"""Pins the oracle (the C restatement of Spar's CPU loops) on the CPU.

The reference ships no tests, fixtures or golden vectors and cannot be built
here (its sources need C++23 `import std`), so each oracle function is checked against
something independent of its own code, chosen so a plausible restatement
mistake (wrong loop order, transposed stride, dropped term, wrong rounding
step) fails:
  * IEEE-754 single/double operations as numpy performs them (one correctly
    rounded operation per element);
  * numpy's sequential accumulation (np.add.accumulate), which fixes the
    summation order of the reference's in-order loops bit for bit;
  * float64 / math.fsum evaluations of the same formulas (closed forms);
  * invariants (sum of probabilities, exp(log p) = p, softmax backward sums
    to zero) and the reference's documented special-case tables;
  * published SplitMix64 output vectors and the committed golden fixtures
    in tests/golden/.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import ops as O
from tests.helpers import assert_bitexact, assert_ulp

F32, F64 = np.float32, np.float64
GOLDEN = Path(__file__).resolve().parent / "golden"


def rnd(seed, shape, dtype=F32, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(dtype)


# ---------------------------------------------------------------- random

def test_splitmix64_published_vectors():
    # SplitMix64 reference outputs (Vigna's splitmix64.c): seed 0 and seed 1234567
    r = O.Random(0)
    assert [r.next_u64() for _ in range(4)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    r = O.Random(1234567)
    assert [r.next_u64() for _ in range(3)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423]


def test_uniform_bits_and_range():
    r1, r2 = O.Random(42), O.Random(42)
    u = r1.uniform((1000,), F32, 0.0, 1.0)
    # uniform_float = (u64 >> 40) / 2^24 (random.cpp:30-33)
    expect = np.array([(r2.next_u64() >> 40) / 16777216.0 for _ in range(1000)], dtype=F32)
    assert_bitexact(u, expect, "uniform_float")
    v = O.Random(3).uniform((100000,), F32, -0.1, 0.1)
    assert v.min() >= -0.1 and v.max() < 0.1
    d = O.Random(5).uniform((10,), F64)
    r = O.Random(5)
    assert_bitexact(d, np.array([(r.next_u64() >> 11) / 2.0 ** 53 for _ in range(10)]), "double")


def test_normal_moments():
    z = O.Random(9).normal((400000,), F64, 0.0, 2.0)
    assert abs(z.mean()) < 0.02 and abs(z.std() - 2.0) < 0.02
    r = O.Random(9)
    u0, u1 = r.uniform_double(), r.uniform_double()
    assert z[0] == 2.0 * (math.sqrt(-2 * math.log(1 - u0)) * math.cos(2 * math.pi * u1))


# ---------------------------------------------------------- elementwise

@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("op,fn", [("add", np.add), ("subtract", np.subtract),
                                   ("multiply", np.multiply), ("divide", np.divide)])
def test_binary_matches_ieee_with_broadcast_and_views(dtype, op, fn):
    a = rnd(1, (5, 7, 9), dtype)
    b = rnd(2, (7, 1), dtype)
    with np.errstate(all="ignore"):
        assert_bitexact(O.binary(a, b, op), fn(a, b), f"{op} broadcast")
        base = rnd(3, (9, 7), dtype)
        assert_bitexact(O.binary(a[1], base.T, op), fn(a[1], base.T), f"{op} transposed view")
        left, right = a[:, 2:5, 0:8:2], a[:, 1:4, 1::2]
        assert_bitexact(O.binary(left, right, op), fn(left, right), f"{op} sliced views")


@pytest.mark.parametrize("op,fn", [("equal", np.equal), ("not_equal", np.not_equal),
                                   ("less", np.less), ("less_equal", np.less_equal),
                                   ("greater", np.greater), ("greater_equal", np.greater_equal)])
def test_compare_truth_tables(op, fn):
    values = np.array([np.nan, -np.inf, -1.0, -0.0, 0.0, 1.0, np.inf], dtype=F32)
    a, b = np.meshgrid(values, values, indexing="ij")
    with np.errstate(invalid="ignore"):
        assert_bitexact(O.binary(a, b, op), fn(a, b).astype(F32), op)


@pytest.mark.parametrize("op,fn", [("add", np.add), ("subtract", np.subtract),
                                   ("multiply", np.multiply), ("divide", np.divide)])
def test_scalar_rounds_double_to_float_first(op, fn):
    a = rnd(4, (1000,))
    for value in (0.1, 1.0 / 3.0, -2.5, 1e-30):
        # scalar.cpp:47: static_cast<float>(value) before the operation
        assert_bitexact(O.scalar(a, op, value), fn(a, F32(value)), f"{op} {value}")


def test_exact_unary_ops():
    a = np.concatenate([rnd(5, (10000,), F32, 10.0), np.array([0.0, -0.0, np.inf, -np.inf], F32)])
    with np.errstate(all="ignore"):
        assert_bitexact(O.unary(a, "negate"), -a, "negate")
        assert_bitexact(O.unary(a, "square"), a * a, "square")
        assert_bitexact(O.unary(a, "reciprocal"), F32(1) / a, "reciprocal")
        b = np.abs(a)
        assert_bitexact(O.unary(b, "sqrt"), np.sqrt(b), "sqrt")


def rounded(f64_values, dtype=F32):
    return np.asarray(f64_values, dtype=np.float64).astype(dtype)


def test_transcendentals_against_double_precision():
    x = rnd(6, (100000,), F32, 4.0)
    x64 = x.astype(np.float64)
    with np.errstate(all="ignore"):
        assert_ulp(O.unary(x, "exp"), rounded(np.exp(x64)), 1, "expf")
        pos = np.abs(x) + F32(1e-6)
        assert_ulp(O.unary(pos, "log"), rounded(np.log(pos.astype(np.float64))), 1, "logf")
        assert_ulp(O.unary(x, "tanh"), rounded(np.tanh(x64)), 2, "tanhf")
        # sigmoid/silu restate unary.cpp:55-61 in float: close to the exact value
        sig = 1.0 / (1.0 + np.exp(-x64))
        assert_ulp(O.unary(x, "sigmoid"), rounded(sig), 3, "sigmoid")
        assert_ulp(O.unary(x, "silu"), rounded(x64 * sig), 4, "silu")


def test_gelu_closed_form():
    from scipy.special import erfc

    x = np.concatenate([rnd(7, (100000,), F32, 4.0), np.array([0.0, -0.0, 30.0, -30.0], F32)])
    x64 = x.astype(np.float64)
    want = rounded(0.5 * x64 * erfc(-x64 / math.sqrt(2.0)))
    assert_ulp(O.unary(x, "gelu"), want, 1, "gelu")
    assert O.unary(np.array([0.0], F32), "gelu")[0] == 0.0
    big = np.array([10.0, 20.0], F32)
    assert_bitexact(O.unary(big, "gelu"), big, "gelu(x) = x for large x")
    d = O.unary(x, "gelu_derivative").astype(np.float64)
    h = 1e-4
    numeric = (0.5 * (x64 + h) * erfc(-(x64 + h) / math.sqrt(2)) -
               0.5 * (x64 - h) * erfc(-(x64 - h) / math.sqrt(2))) / (2 * h)
    assert np.max(np.abs(d - numeric)) < 1e-6


# ------------------------------------------------------------ reductions

@pytest.mark.parametrize("dtype", [F32, F64])
def test_full_sum_is_sequential(dtype):
    x = rnd(8, (100003,), dtype)
    assert O.full_reduce(x, "sum") == np.add.accumulate(x, dtype=dtype)[-1]
    n = dtype(x.size)
    assert O.full_reduce(x, "mean") == np.add.accumulate(x, dtype=dtype)[-1] / n
    exact = math.fsum(x.astype(np.float64))
    assert abs(float(O.full_reduce(x, "sum")) - exact) < 1e-6 * math.sqrt(x.size) * \
        math.sqrt(float(np.sum(x.astype(np.float64) ** 2)))
    view = rnd(9, (300, 200), dtype).T
    assert O.full_reduce(view, "sum") == np.add.accumulate(view.reshape(-1), dtype=dtype)[-1]


def test_full_max_rules():
    assert O.full_reduce(np.array([1, 3, 2], F32), "max") == 3
    assert np.isnan(O.full_reduce(np.array([1, np.nan, 5], F32), "max"))
    z = O.full_reduce(np.array([-0.0, 0.0, -1.0], F32), "max")
    assert z == 0 and np.signbit(z)  # first of the equal zeros
    assert O.full_reduce(np.array([-np.inf, -np.inf], F32), "max") == -np.inf


def test_axis_sum_order_matches_sequential_accumulation():
    x = rnd(10, (6, 40, 50))
    assert_bitexact(O.axis_sum(x, [0]), np.add.accumulate(x, axis=0)[-1], "axis 0")
    assert_bitexact(O.axis_sum(x, [2]), np.add.accumulate(x, axis=2)[..., -1], "axis 2")
    # axes {0, 2}: each output accumulates its elements in (a, c) order
    seq = np.add.accumulate(x.transpose(1, 0, 2).reshape(40, -1), axis=1)[:, -1]
    assert_bitexact(O.axis_sum(x, [0, 2]), seq, "axes 0,2")
    t = x[1].T  # a transposed view: logical order, not storage order
    assert_bitexact(O.axis_sum(t, [1]), np.add.accumulate(np.ascontiguousarray(t), axis=1)[:, -1],
                    "view")


def test_axis_max_argmax_first_occurrence():
    x = rnd(11, (30, 40))
    x[3, 7] = x[3, 20] = 99.0
    x[5, :] = 0.0
    x[5, 4] = -0.0
    x[8, 6] = np.nan
    x[8, 9] = np.nan
    values, indices = O.axis_max(x, [1])
    assert_bitexact(indices, np.argmax(x, axis=1), "argmax = numpy first occurrence")
    assert indices[3] == 7 and indices[8] == 6 and indices[5] == 0
    assert_bitexact(values[[0, 1, 2, 3]], np.max(x[[0, 1, 2, 3]], axis=1), "max values")
    values0, indices0 = O.axis_max(x, [0])
    assert_bitexact(indices0, np.argmax(x, axis=0), "argmax axis 0")


def test_reduce_gradient_brute_force():
    g = rnd(12, (3, 4, 5))
    assert_bitexact(O.reduce_gradient(g, (5,)), np.add.accumulate(g.reshape(12, 5), axis=0)[-1],
                    "leading axes")
    assert_bitexact(O.reduce_gradient(g, (4, 1)), np.add.accumulate(
        g.transpose(1, 0, 2).reshape(4, 15), axis=1)[:, -1].reshape(4, 1), "trailing 1")
    assert_bitexact(O.reduce_gradient(g, (3, 1, 5)), np.add.accumulate(g, axis=1)[:, -1:, :],
                    "middle 1")
    assert_bitexact(O.reduce_gradient(g, (3, 4, 5)), g + F32(0), "identity")
    assert O.reduce_gradient(g, ()).shape == ()


def test_strided_copy_is_numpy_copy():
    base = rnd(13, (7, 11, 13))
    for view in (base.transpose(2, 0, 1), base[1:6, ::2, 3:], np.broadcast_to(base[0, 0], (4, 13))):
        assert_bitexact(O.strided_copy(view), np.ascontiguousarray(view), "copy")


# ---------------------------------------------------------------- softmax

def test_softmax_closed_form_and_invariants():
    x = rnd(14, (20, 300), F32, math.sqrt(2))
    p, und = O.softmax_axis(x, 1)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    exact = e / e.sum(axis=1, keepdims=True)
    assert np.max(np.abs(p - exact) / exact) < 1e-5
    assert not und.any()
    assert np.allclose(p.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)
    lp, _ = O.log_softmax(x, 1)
    assert np.allclose(np.exp(lp.astype(np.float64)), p, rtol=1e-5)
    p0, _ = O.softmax_axis(x, 0)
    assert_bitexact(p0, O.softmax_axis(np.ascontiguousarray(x.T), 1)[0].T.copy(), "axis 0")
    # the full softmax of a row equals its axis softmax (same loop order)
    assert_bitexact(O.softmax_full(x[3]), p[3], "full vs axis")


def test_softmax_special_case_table():
    inf, nan = np.inf, np.nan
    x = np.array([[nan, 1, 2], [-inf, -inf, -inf], [inf, 0, inf], [inf, -inf, 1]], F32)
    p, und = O.softmax_axis(x, 1)
    assert np.isnan(p[0]).all() and np.isnan(p[1]).all()
    assert_bitexact(p[2], np.array([0.5, 0, 0.5], F32), "two +inf")
    assert_bitexact(p[3], np.array([1, 0, 0], F32), "one +inf")
    assert list(und) == [1, 1, 1, 1]
    lp, und = O.log_softmax(x, 1)
    assert_bitexact(lp[2], np.array([-np.log(F32(2)), -inf, -np.log(F32(2))], F32), "log +inf")
    assert list(und) == [1, 1, 1, 1]
    assert O.softmax_full_undefined(np.array([-inf, -inf], F32))
    assert not O.softmax_full_undefined(np.array([-inf, 0.0], F32))


def test_softmax_backward_closed_form():
    x = rnd(15, (10, 64), F64)
    g = rnd(16, (10, 64), F64)
    p, und = O.softmax_axis(x, 1)
    dx = O.softmax_axis_backward(g, p, und, 1)
    jac = p * (g - np.sum(g * p, axis=1, keepdims=True))
    assert np.allclose(dx, jac, atol=1e-14)
    assert np.allclose(dx.sum(axis=1), 0, atol=1e-12)
    lp, und = O.log_softmax(x, 1)
    dl = O.log_softmax_backward(g, lp, und, 1)
    assert np.allclose(dl, g - np.exp(lp) * g.sum(axis=1, keepdims=True), atol=1e-13)
    und[3] = 1
    assert np.isnan(O.softmax_axis_backward(g, p, und, 1)[3]).all()


# ------------------------------------------------------ committed fixtures

def test_golden_fixtures():
    """Small vectors committed under tests/golden/ (inputs and expected
    outputs written by tests/golden/make_golden.py from float64 closed forms
    and exact integer arithmetic, independent of the oracle's loops)."""
    data = json.loads((GOLDEN / "vectors.json").read_text())
    for case in data["cases"]:
        a = np.array(case["a"], dtype=case["dtype"]).reshape(case["shape_a"])
        if case["kind"] == "binary":
            b = np.array(case["b"], dtype=case["dtype"]).reshape(case["shape_b"])
            got = O.binary(a, b, case["op"])
        elif case["kind"] == "unary":
            got = O.unary(a, case["op"])
        elif case["kind"] == "axis_sum":
            got = O.axis_sum(a, case["axes"])
        elif case["kind"] == "softmax":
            got = O.softmax_axis(a, case["axis"])[0]
        else:
            raise AssertionError(case["kind"])
        want = np.array(case["expected"], dtype=case["dtype"]).reshape(got.shape)
        if case["tolerance_ulp"] == 0:
            assert_bitexact(got, want, case["name"])
        else:
            assert_ulp(got, want, case["tolerance_ulp"], case["name"])


def _closed_form_lp(x):
    x = x.astype(np.float64)
    z = x - x.max(axis=-1, keepdims=True)
    return z - np.log(np.exp(z).sum(axis=-1, keepdims=True))


@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_cross_entropy_restatement_closed_form(reduction):
    """loss_i = -lp[i, t_i] and dlogits = (softmax - onehot) * dreduce, from
    float64 closed forms; a dropped sign or a wrong target index fails."""
    import oracle.reference as R

    rng = np.random.default_rng(70)
    x = (rng.standard_normal((6, 7, 11)) * 2).astype(np.float32)
    t = rng.integers(0, 11, (6, 7)).astype(np.int32)
    logits = R.RTensor.of(x, requires_grad=True)
    loss = R.cross_entropy(logits, t, reduction)
    lp = _closed_form_lp(x)
    per = -np.take_along_axis(lp, t[..., None].astype(np.int64), -1)[..., 0]
    want = {"none": per, "sum": per.sum(), "mean": per.mean()}[reduction]
    assert np.allclose(loss.numpy(), want, rtol=2e-6, atol=2e-6)
    R.sum(loss).backward() if reduction == "none" else loss.backward()
    onehot = np.zeros_like(lp)
    np.put_along_axis(onehot, t[..., None].astype(np.int64), 1.0, -1)
    scale = 1.0 / t.size if reduction == "mean" else 1.0
    assert np.allclose(logits.grad().numpy(), (np.exp(lp) - onehot) * scale, rtol=2e-5, atol=1e-7)


def test_language_model_cross_entropy_restatement_shifts_targets():
    import oracle.reference as R

    rng = np.random.default_rng(71)
    x = rng.standard_normal((3, 5, 9)).astype(np.float32)
    ids = rng.integers(0, 9, (3, 5)).astype(np.int64)
    logits = R.RTensor.of(x, requires_grad=True)
    loss = R.language_model_cross_entropy(logits, ids, "none")
    lp = _closed_form_lp(x)
    want = -np.take_along_axis(lp[:, :-1], ids[:, 1:, None], -1)[..., 0]
    assert loss.shape == (3, 4) and np.allclose(loss.numpy(), want, rtol=2e-6, atol=2e-6)
    R.sum(loss).backward()
    grad = logits.grad().numpy()
    assert not grad[:, -1].any(), "the last position has no target"
    onehot = np.zeros_like(lp[:, :-1])
    np.put_along_axis(onehot, ids[:, 1:, None], 1.0, -1)
    assert np.allclose(grad[:, :-1], np.exp(lp[:, :-1]) - onehot, rtol=2e-5, atol=1e-7)


def test_cross_entropy_restatement_errors():
    import oracle.reference as R

    logits = R.RTensor.of(np.zeros((2, 3), np.float32))
    with pytest.raises(IndexError):
        R.cross_entropy(logits, np.array([0, 3], np.int64))
    with pytest.raises(IndexError):
        R.cross_entropy(logits, np.array([-1, 0], np.int32))
    with pytest.raises(ValueError):
        R.cross_entropy(logits, np.array([0.0, 1.0], np.float32))
    with pytest.raises(ValueError):
        R.cross_entropy(logits, np.array([0, 1, 2], np.int64))


# ------------------------------------------------ optimizer and gradient norm
#
# The reference has no fixtures for these either.  AdamW is pinned against
# torch.optim.AdamW in float64 (the same decoupled-decay algorithm written
# with different but mathematically equal operations) and closed forms; the
# norm accumulator against numpy's L2 norm, exact maxima and the documented
# special cases; scaling against exact rational arithmetic.

def _torch_adamw(p, grads, lr, b1, b2, eps, wd):
    import torch

    t = torch.tensor(p, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.AdamW([t], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd,
                            foreach=False)
    for g in grads:
        t.grad = torch.tensor(g, dtype=torch.float64)
        opt.step()
    return t.detach().numpy()


@pytest.mark.parametrize("lr,b1,b2,eps,wd", [(1e-3, 0.9, 0.999, 1e-8, 0.01),
                                             (0.05, 0.5, 0.9, 1e-6, 0.1),
                                             (0.01, 0.0, 0.0, 1e-3, 0.0)])
def test_adamw_restatement_matches_torch_float64(lr, b1, b2, eps, wd):
    rng = np.random.default_rng(90)
    p0 = rng.standard_normal(257)
    grads = [rng.standard_normal(257) * 10.0 ** rng.integers(-3, 3) for _ in range(7)]
    p = p0.copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    for step, g in enumerate(grads, start=1):
        O.adamw(p, g, m, v, lr, b1, b2, eps, wd, O.adamw_correction(b1, step),
                O.adamw_correction(b2, step))
    want = _torch_adamw(p0, grads, lr, b1, b2, eps, wd)
    scale = np.abs(p0) + lr * len(grads)
    assert np.all(np.abs(p - want) <= 1e-13 * scale), np.max(np.abs(p - want) / scale)


def test_adamw_restatement_closed_forms():
    rng = np.random.default_rng(91)
    lr, b1, b2, eps, wd = 0.01, 0.9, 0.999, 1e-8, 0.1
    # step 1 from zero moments: m_hat = g, v_hat = g^2, so p -= lr g / (|g| + eps)
    p0 = rng.standard_normal(64)
    g = rng.standard_normal(64)
    p, m, v = p0.copy(), np.zeros(64), np.zeros(64)
    O.adamw(p, g, m, v, lr, b1, b2, eps, wd, O.adamw_correction(b1, 1), O.adamw_correction(b2, 1))
    want = p0 * (1 - lr * wd) - lr * g / (np.abs(g) + eps)
    assert np.allclose(p, want, rtol=0, atol=1e-15)
    assert np.allclose(m, (1 - b1) * g, rtol=1e-15, atol=0)
    assert np.allclose(v, (1 - b2) * g * g, rtol=1e-15, atol=0)
    # a constant gradient keeps m_hat = g and v_hat = g^2 at every step, so
    # each step moves by lr sign(g) (bias correction exact in the limit)
    p, m, v = p0.copy(), np.zeros(64), np.zeros(64)
    for step in range(1, 21):
        O.adamw(p, g, m, v, lr, b1, b2, eps, 0.0, O.adamw_correction(b1, step),
                O.adamw_correction(b2, step))
    assert np.allclose(p, p0 - 20 * lr * g / (np.abs(g) + eps), rtol=0, atol=1e-12)
    # zero gradients: only the decoupled decay acts, p_t = p (1 - lr wd)^t
    p, m, v = p0.copy(), np.zeros(64), np.zeros(64)
    for step in range(1, 6):
        O.adamw(p, np.zeros(64), m, v, lr, b1, b2, eps, wd, O.adamw_correction(b1, step),
                O.adamw_correction(b2, step))
    assert np.allclose(p, p0 * (1 - lr * wd) ** 5, rtol=1e-15, atol=0)
    assert not m.any() and not v.any()
    assert O.adamw_correction(0.9, 3) == 1 - 0.9 ** 3


def test_adamw_restatement_rounds_moments_to_float32():
    """For float32 parameters the moments are stored as float32 and the step
    reads them back: the result equals the float64 step computed from the
    float32-rounded moments, and differs from an unrounded float64 update."""
    rng = np.random.default_rng(92)
    p = rng.standard_normal(512).astype(F32)
    g = rng.standard_normal(512).astype(F32)
    m = rng.standard_normal(512).astype(F32) * F32(0.1)
    v = np.abs(rng.standard_normal(512)).astype(F32) * F32(0.01)
    lr, b1, b2, eps, wd, c1, c2 = 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.5, 0.25
    p32, m32, v32 = p.copy(), m.copy(), v.copy()
    O.adamw(p32, g, m32, v32, lr, b1, b2, eps, wd, c1, c2)
    g64 = g.astype(F64)
    m_want = (b1 * m.astype(F64) + (1 - b1) * g64).astype(F32)
    v_want = (b2 * v.astype(F64) + (1 - b2) * g64 * g64).astype(F32)
    assert_bitexact(m32, m_want, "float32 first moment")
    assert_bitexact(v32, v_want, "float32 second moment")
    step = lr * (m_want.astype(F64) / c1) / (np.sqrt(v_want.astype(F64) / c2) + eps)
    assert_bitexact(p32, (p.astype(F64) * (1 - lr * wd) - step).astype(F32), "float32 parameter")


@pytest.mark.parametrize("dtype", [F32, F64])
def test_sum_squares_restatement(dtype):
    rng = np.random.default_rng(93)
    for n in (1, 2, 17, 10000):
        x = (rng.standard_normal(n) * 10.0 ** rng.integers(-5, 5, n)).astype(dtype)
        acc = O.SumSquares().add(x)
        assert acc.scale == float(np.max(np.abs(x)))
        assert acc.scaled_sum_squares >= 1.0
        want = float(np.linalg.norm(x.astype(F64)))
        assert abs(acc.norm() - want) <= 1e-13 * want
    # squares that overflow or underflow double: the scaled form stays exact
    for magnitude in (1e300, 1e-300):
        x = rng.standard_normal(1000) * magnitude
        want = float(np.linalg.norm(x / magnitude)) * magnitude
        assert abs(O.SumSquares().add(x).norm() - want) <= 1e-13 * want
    # special cases (gradients.cpp:79-87): NaN beats infinity, zeros and empty give 0
    assert math.isnan(O.SumSquares().add(np.array([1.0, np.inf, np.nan], dtype)).norm())
    inf = O.SumSquares().add(np.array([1.0, -np.inf, 2.0], dtype))
    assert inf.norm() == math.inf and inf.has_infinity and not inf.has_nan
    assert inf.scale == 2.0 and inf.scaled_sum_squares == 1.25
    assert O.SumSquares().add(np.zeros(5, dtype)).norm() == 0.0
    empty = O.SumSquares().add(np.zeros(0, dtype))
    assert (empty.scale, empty.scaled_sum_squares, empty.norm()) == (0.0, 1.0, 0.0)
    # combining two halves' accumulators matches feeding all elements
    x = rng.standard_normal(999).astype(dtype)
    a, b = O.SumSquares().add(x[:400]), O.SumSquares().add(x[400:])
    a.combine(b.scale, b.scaled_sum_squares, b.has_infinity, b.has_nan)
    whole = O.SumSquares().add(x)
    assert a.scale == whole.scale
    assert abs(a.norm() - whole.norm()) <= 1e-14 * whole.norm()


def test_scale_restatement_rounds_through_double():
    from fractions import Fraction

    rng = np.random.default_rng(94)
    x = rng.standard_normal(300).astype(F32)
    for factor in (0.1, 1.0 / 3.0, 2.0 ** -7, 12345.678):
        got = x.copy()
        O.scale(got, factor)
        want = np.array([np.float32(float(Fraction(float(v)) * Fraction(factor))) for v in x], F32)
        assert_bitexact(got, want, f"scale by {factor}")
    got = x.astype(F64)
    O.scale(got, 2.0 ** 10)
    assert_bitexact(got, x.astype(F64) * 1024.0, "power-of-two scale is exact")


def test_clip_grad_norm_restatement():
    import oracle.reference as R

    rng = np.random.default_rng(95)
    grads = [rng.standard_normal(100).astype(F32), None, rng.standard_normal((3, 7)).astype(F32)]
    total = float(np.sqrt(sum(np.sum(g.astype(F64) ** 2) for g in grads if g is not None)))
    assert abs(R.global_grad_norm(grads) - total) <= 1e-13 * total
    kept = [None if g is None else g.copy() for g in grads]
    assert R.clip_grad_norm(kept, 2 * total) == (R.global_grad_norm(grads), 1.0, False)
    norm, factor, clipped = R.clip_grad_norm(kept, 1.0)
    assert clipped and factor == 1.0 / norm
    assert abs(R.global_grad_norm(kept) - 1.0) <= 1e-6
    with pytest.raises(ValueError):
        R.clip_grad_norm(kept, -1.0)
    with pytest.raises(RuntimeError):
        R.clip_grad_norm([np.array([np.nan], F32)], 1.0)
