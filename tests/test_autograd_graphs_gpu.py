"""Random small graphs through the engine with its hand-overs on and off.

backward() may hand a narrow's gradient down a chain of narrows and embed it
once, let a fused norm write its input's gradient straight into the box of
the chain base's gradient, and hand a product's gradient to a norm as
(factor, value) instead of materialising it (autograd.cpp, contract points
5 and 6).  spar.set_autograd_hand_overs(False) makes every rule run in its
plain form.  The contract is that both give the same bits; these graphs mix
narrow chains (some narrowed views used twice, so their gradient is not
handed down), transposes, elementwise ops with broadcasting, row means,
layer_norm on every kind of view, and products with constants, from seeded
random recipes, and compare every leaf gradient bit for bit.
"""
import numpy as np
import pytest

from tests.helpers import assert_bitexact

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module")
def sp():
    from spar_amd import spar

    if spar.hip_device_count() < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    yield spar
    spar.set_autograd_hand_overs(True)


def recipe(seed):
    """A graph as a list of steps over value indices; value 0 is the base
    leaf.  Returns (base shape, steps, loss kind)."""
    rng = np.random.default_rng(seed)
    base = (int(rng.integers(6, 40)), int(rng.integers(6, 72)))
    shapes = [base]
    steps = []

    def pick(two_d=True):
        candidates = [k for k, s in enumerate(shapes) if not two_d or len(s) == 2]
        return int(rng.choice(candidates))

    for _ in range(int(rng.integers(3, 10))):
        kind = rng.choice(["narrow", "narrow", "narrow2", "transpose", "binary", "constant",
                           "layer_norm", "layer_norm", "center", "unary"])
        v = pick()
        rows, cols = shapes[v]
        if kind in ("narrow", "narrow2"):
            out = shapes[v]
            axes = [int(rng.integers(0, 2))] if kind == "narrow" else [0, 1]
            windows = []
            for axis in axes:
                extent = out[axis]
                if extent < 2:
                    continue
                length = int(rng.integers(1, extent))
                start = int(rng.integers(0, extent - length + 1))
                windows.append((axis, start, length))
                out = tuple(length if a == axis else d for a, d in enumerate(out))
            if not windows:
                continue
            steps.append(("narrow", v, windows))
            shapes.append(out)
        elif kind == "transpose":
            steps.append(("transpose", v))
            shapes.append((cols, rows))
        elif kind == "binary":
            same = [k for k, s in enumerate(shapes) if s == shapes[v]]
            w = int(rng.choice(same))  # possibly v itself
            steps.append(("binary", v, w, str(rng.choice(["add", "subtract", "multiply"]))))
            shapes.append(shapes[v])
        elif kind == "constant":
            steps.append(("constant", v, int(rng.integers(0, 1 << 30))))
            shapes.append(shapes[v])
        elif kind == "layer_norm":
            steps.append(("layer_norm", v, int(rng.integers(0, 1 << 30))))
            shapes.append(shapes[v])
        elif kind == "center":
            steps.append(("center", v))  # v - mean(v, 1, keepdim)
            shapes.append(shapes[v])
        else:
            steps.append(("unary", v, str(rng.choice(["square", "exp", "negate"]))))
            shapes.append(shapes[v])
    if rng.random() < 0.5:
        # end with a chain of narrows of the base into a layer_norm: the
        # norm may write its gradient into the chain base's box
        v, out, windows = 0, base, []
        for axis in (0, 1, int(rng.integers(0, 2))):
            if out[axis] >= 2:
                length = int(rng.integers(1, out[axis]))
                start = int(rng.integers(0, out[axis] - length + 1))
                windows.append((axis, start, length))
                out = tuple(length if a == axis else d for a, d in enumerate(out))
        if windows:
            steps.append(("narrow", v, windows))
            shapes.append(out)
            steps.append(("layer_norm", len(shapes) - 1, int(rng.integers(0, 1 << 30))))
            shapes.append(out)
    loss = str(rng.choice(["sum", "constant", "constant", "mean"]))
    return base, steps, loss, int(rng.integers(0, 1 << 30))


def run(sp, seed, hand_overs):
    base_shape, steps, loss_kind, loss_seed = recipe(seed)
    device, cpu = sp.Device.hip(0), sp.Device.cpu()
    rng = np.random.default_rng(seed + 1000)

    def leaf(array, grad=True):
        t = sp.Tensor.from_numpy(np.ascontiguousarray(array, dtype=F32)).to(device)
        if grad:
            t.set_requires_grad(True)
        return t

    leaves = [leaf(rng.standard_normal(base_shape))]
    values = [leaves[0]]
    for step in steps:
        kind, v = step[0], values[step[1]]
        if kind == "narrow":
            for axis, start, length in step[2]:
                v = v.narrow(axis, start, length)
            values.append(v)
        elif kind == "transpose":
            values.append(v.transpose(0, 1))
        elif kind == "binary":
            values.append(getattr(sp, step[3])(v, values[step[2]]))
        elif kind == "constant":
            c = np.random.default_rng(step[2]).standard_normal(tuple(v.shape)).astype(F32)
            values.append(sp.multiply(v, leaf(c, grad=False)))
        elif kind == "layer_norm":
            p = np.random.default_rng(step[2])
            n = tuple(v.shape)[1]
            gamma, beta = leaf(p.uniform(0.5, 1.5, n)), leaf(p.uniform(-0.1, 0.1, n))
            leaves += [gamma, beta]
            values.append(sp.layer_norm(v, gamma, beta, 1e-5))
        elif kind == "center":
            values.append(sp.subtract(v, sp.mean(v, [1], True)))
        else:
            op = {"square": sp.square, "exp": sp.exp, "negate": sp.negate}[step[2]]
            if not v.is_contiguous():  # unary ops take contiguous inputs, as the reference's
                v = v.contiguous()
            values.append(op(v))
    final = values[-1]
    if loss_kind == "sum":
        loss = sp.sum(final, None, False)
    elif loss_kind == "mean":
        loss = sp.mean(final, None, False)
    else:
        c = np.random.default_rng(loss_seed).standard_normal(tuple(final.shape)).astype(F32)
        loss = sp.sum(sp.multiply(final, leaf(c, grad=False)), None, False)
    sp.set_autograd_hand_overs(hand_overs)
    try:
        before = sp.autograd_counters()
        loss.backward()
        after = sp.autograd_counters()
    finally:
        sp.set_autograd_hand_overs(True)
    taken = {k: after[k] - before[k] for k in ("window_fusions", "placed_gradients",
                                               "scaled_gradients")}
    grads = [t.grad().to(cpu).numpy() if t.has_grad else None for t in leaves]
    return grads, taken


def test_random_graphs_same_bits_with_and_without_hand_overs(sp):
    taken_total = {"window_fusions": 0, "placed_gradients": 0, "scaled_gradients": 0}
    for seed in range(120):
        fused, taken = run(sp, seed, True)
        plain, plain_taken = run(sp, seed, False)
        assert not any(plain_taken.values()), f"graph {seed}: a hand-over ran while they were off"
        for key, count in taken.items():
            taken_total[key] += count
        assert len(fused) == len(plain)
        for k, (a, b) in enumerate(zip(fused, plain)):
            assert (a is None) == (b is None), f"graph {seed} leaf {k}: gradient presence"
            if a is not None:
                assert_bitexact(a, b, f"graph {seed} leaf {k} {recipe(seed)[1]}")
    # the recipes exercise every hand-over, not only the plain paths
    assert all(count >= 5 for count in taken_total.values()), taken_total
