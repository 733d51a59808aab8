"""Public tensor/ops API on HIP tensors against the oracle's restatement of
Spar's CPU path (oracle.reference), including autograd.

Parity classes (tests/helpers.py): elementwise, broadcast, layout, compare,
argmax and max are bit-exact; transcendentals <= 2 ulp (float32);
reductions red(N).  Gradients that pass only through elementwise ops are
bit-exact; gradients that pass through a reduction are compared with the
red bound of that reduction.
"""
import numpy as np
import pytest

import oracle.reference as R
from oracle import ops as C
from tests.helpers import assert_bitexact, assert_red, assert_ulp

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module")
def sp():
    from spar_amd import spar

    if spar.hip_device_count() < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    return spar


def hip_tensor(sp, array, requires_grad=False):
    t = sp.Tensor.from_numpy(np.ascontiguousarray(array)).to(sp.Device.hip(0))
    if requires_grad:
        t.set_requires_grad(True)
    return t


def host(sp, tensor):
    return tensor.to(sp.Device.cpu()).numpy()


def normal(seed, shape, scale=1.0, dtype=F32):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(dtype)


# ------------------------------------------------------------ transfers

def test_round_trip_and_views(sp):
    x = normal(1, (37, 53))
    t = hip_tensor(sp, x)
    assert t.device == sp.Device.hip(0)
    assert_bitexact(host(sp, t), x, "round trip")
    assert_bitexact(host(sp, t.transpose(0, 1)), x.T.copy(), "transpose to host")
    assert_bitexact(host(sp, t.narrow(0, 3, 20).narrow(1, 5, 40)), x[3:23, 5:45].copy(), "narrow")
    assert_bitexact(host(sp, t.transpose(0, 1).contiguous()), x.T.copy(), "contiguous")
    cpu_view = sp.Tensor.from_numpy(x).transpose(0, 1)
    assert_bitexact(host(sp, cpu_view.to(sp.Device.hip(0))), x.T.copy(), "host view upload")
    e = hip_tensor(sp, x[0]).expand([4, 53])
    assert e.strides == [0, 1]
    assert_bitexact(host(sp, e), np.broadcast_to(x[0], (4, 53)).copy(), "expand")


def test_factories_on_device(sp):
    dev = sp.Device.hip(0)
    assert np.all(host(sp, sp.zeros([5, 7], sp.DType.float32, dev)) == 0)
    assert np.all(host(sp, sp.ones([5, 7], sp.DType.float64, dev)) == 1)
    assert np.all(host(sp, sp.full([3], 2.5, sp.DType.float32, dev)) == 2.5)
    assert np.all(host(sp, sp.full([3], 7, sp.DType.int64, dev)) == 7)


def test_random_uniform_device_matches_host(sp):
    r_host, r_dev = sp.Random(5), sp.Random(5)
    a = sp.random_uniform([1000], sp.DType.float32, r_host, -2.0, 3.0)
    b = sp.random_uniform([1000], sp.DType.float32, r_dev, -2.0, 3.0, sp.Device.hip(0))
    assert_bitexact(host(sp, b), a.numpy(), "device uniform")
    assert r_host.state == r_dev.state
    ref = C.Random(5).uniform((1000,), F32, -2.0, 3.0)
    assert_bitexact(a.numpy(), ref, "host uniform vs oracle")


# ----------------------------------------------------------- elementwise

BINARY = ["add", "subtract", "multiply", "divide"]
COMPARE = ["equal", "not_equal", "less", "less_equal", "greater", "greater_equal"]


@pytest.mark.parametrize("op", BINARY + COMPARE)
@pytest.mark.parametrize("shapes", [((6, 8, 12), (12,)), ((6, 8, 12), (6, 1, 12)),
                                    ((6, 1, 12), (1, 8, 1)), ((5,), (5,)), ((), (3, 4))])
def test_binary_broadcast_api(sp, op, shapes):
    a = normal(2, shapes[0])
    b = normal(3, shapes[1])
    if op in COMPARE:
        b = np.where(np.random.default_rng(9).random(b.shape) < 0.3,
                     np.broadcast_to(a.reshape(-1)[0], b.shape), b).astype(F32)
    got = host(sp, getattr(sp, op)(hip_tensor(sp, a), hip_tensor(sp, b)))
    want = C.binary(a, b, op)
    assert_bitexact(got, want, op)


def test_binary_on_views(sp):
    base = normal(4, (64, 96))
    other = normal(5, (96, 64))
    tb, to = hip_tensor(sp, base), hip_tensor(sp, other)
    got = host(sp, sp.subtract(tb.transpose(0, 1), to))
    assert_bitexact(got, C.binary(base.T, other, "subtract"), "transposed left")
    got = host(sp, sp.multiply(tb.narrow(0, 10, 30), tb.narrow(0, 20, 30)))
    assert_bitexact(got, C.binary(base[10:40], base[20:50], "multiply"), "narrowed")


def test_binary_errors(sp):
    a = hip_tensor(sp, normal(1, (3, 4)))
    b = hip_tensor(sp, normal(1, (5, 4)))
    with pytest.raises(ValueError):
        sp.add(a, b)
    with pytest.raises(ValueError):
        sp.add(a, hip_tensor(sp, normal(1, (3, 4), dtype=np.float64)))
    with pytest.raises(ValueError):
        sp.add(a, sp.Tensor.from_numpy(normal(1, (3, 4))))
    with pytest.raises(ValueError):
        sp.add(hip_tensor(sp, np.arange(4, dtype=np.int64)), hip_tensor(sp, np.arange(4, dtype=np.int64)))
    x = hip_tensor(sp, normal(1, (3, 4)), requires_grad=True)
    with pytest.raises(sp.LogicError):
        sp.less(x, a)


@pytest.mark.parametrize("op,value", [("add_scalar", 0.1), ("subtract_scalar", 3.0),
                                      ("multiply_scalar", -1.5), ("divide_scalar", 7.0)])
def test_scalar_api(sp, op, value):
    x = normal(6, (33, 7))
    got = host(sp, getattr(sp, op)(hip_tensor(sp, x), value))
    assert_bitexact(got, C.scalar(x, op.split("_")[0], value), op)


def test_scalar_errors(sp):
    x = hip_tensor(sp, normal(6, (4, 5)))
    with pytest.raises(OverflowError):
        sp.add_scalar(x, 1e39)
    with pytest.raises(ValueError):
        sp.add_scalar(x.transpose(0, 1), 1.0)
    sp.add_scalar(x, float("inf"))  # non-finite scalars are allowed


@pytest.mark.parametrize("op", ["negate", "square", "reciprocal", "exp", "log", "sqrt", "sigmoid",
                                "silu", "tanh", "gelu"])
def test_unary_api(sp, op):
    x = normal(7, (257, 31), 3.0)
    if op in ("log", "sqrt"):
        x = np.abs(x) + F32(1e-3)
    got = host(sp, getattr(sp, op)(hip_tensor(sp, x)))
    want = C.unary(x, op)
    if op in ("negate", "square", "reciprocal", "sqrt"):
        assert_bitexact(got, want, op)
    else:
        assert_ulp(got, want, 2, op)
    with pytest.raises(ValueError):
        getattr(sp, op)(hip_tensor(sp, x).transpose(0, 1))


# ------------------------------------------------------------ reductions

def red_norm(x, axes):
    return np.sqrt(C.axis_sum(x.astype(np.float64) ** 2, axes))


@pytest.mark.parametrize("axes,keepdim", [((0,), False), ((1,), True), ((0, 2), False),
                                          ((1, 2), True), ((0, 1, 2), False)])
def test_sum_mean_axes(sp, axes, keepdim):
    x = normal(8, (12, 40, 66))
    t = hip_tensor(sp, x)
    n = int(np.prod([x.shape[a] for a in axes]))
    s = sp.sum(t, list(axes), keepdim)
    expect_shape = tuple(1 if (i in axes) else d for i, d in enumerate(x.shape) if keepdim or i not in axes)
    assert s.shape == expect_shape
    assert_red(host(sp, s).reshape(-1), C.axis_sum(x, axes).reshape(-1), n,
               red_norm(x, axes).reshape(-1), "sum")
    m = sp.mean(t, list(axes), keepdim)
    want = C.scalar(C.axis_sum(x, axes).reshape(-1), "divide", float(n))
    assert_red(host(sp, m).reshape(-1), want, n, red_norm(x, axes).reshape(-1) / n, "mean")


def test_full_reductions_and_views(sp):
    x = normal(9, (300, 257))
    t = hip_tensor(sp, x)
    norm = float(np.sqrt(np.sum(x.astype(np.float64) ** 2)))
    assert_red(host(sp, sp.sum(t)), C.full_reduce(x, "sum"), x.size, norm, "sum")
    assert_red(host(sp, sp.mean(t)), C.full_reduce(x, "mean"), x.size, norm / x.size, "mean")
    assert_bitexact(host(sp, sp.reduce_max(t)), np.array(C.full_reduce(x, "max")), "reduce_max")
    tt = t.transpose(0, 1)
    assert_red(host(sp, sp.sum(tt)), C.full_reduce(x.T, "sum"), x.size, norm, "sum of view")
    assert_red(host(sp, sp.sum(tt, 0)), C.axis_sum(x.T, [0]), 257, red_norm(x.T, [0]), "axis of view")


def test_max_argmax_api(sp):
    x = normal(10, (20, 33))
    x[3, 5] = x[3, 9] = 50.0
    x[7, 2] = np.nan
    t = hip_tensor(sp, x)
    for axis in (0, 1):
        values, indices = C.axis_max(x, [axis])
        assert_bitexact(host(sp, sp.max(t, axis)), values, "max")
        got = sp.argmax(t, axis, True)
        assert got.dtype == sp.DType.int64
        assert_bitexact(host(sp, got).reshape(-1), indices, "argmax")
    with pytest.raises(sp.LogicError):
        sp.reduce_max(hip_tensor(sp, x, requires_grad=True))


def test_reduction_errors(sp):
    t = hip_tensor(sp, normal(1, (3, 4)))
    with pytest.raises(ValueError):
        sp.sum(t, [])
    with pytest.raises(IndexError):
        sp.sum(t, [2])
    with pytest.raises(ValueError):
        sp.sum(t, [1, 1])
    with pytest.raises(ValueError):
        sp.mean(hip_tensor(sp, np.zeros((0, 3), F32)))
    with pytest.raises(ValueError):
        sp.reduce_max(hip_tensor(sp, np.zeros((0,), F32)))
    assert host(sp, sp.sum(hip_tensor(sp, np.zeros((0, 3), F32)), [0])).tolist() == [0, 0, 0]


# --------------------------------------------------------------- softmax

@pytest.mark.parametrize("axis", [None, 0, 1])
def test_softmax_api(sp, axis):
    x = normal(11, (24, 50), np.sqrt(2))
    t = hip_tensor(sp, x)
    got = host(sp, sp.softmax(t, axis))
    want = C.softmax_full(x) if axis is None else C.softmax_axis(x, axis)[0]
    n = x.size if axis is None else x.shape[axis]
    bound = (4 * np.finfo(F32).eps + 1e-6 * np.sqrt(n)) * np.abs(want) + np.finfo(F32).tiny
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)
    lgot = host(sp, sp.log_softmax(t, axis))
    lwant = C.log_softmax(x, axis)[0]
    err = np.abs(lgot.astype(np.float64) - lwant)
    assert np.all(err <= 1e-6 * np.sqrt(n) + 4 * np.finfo(F32).eps * (np.abs(lwant) + np.log(n) + 1))


def test_softmax_errors(sp):
    t = hip_tensor(sp, normal(1, (3, 4)))
    with pytest.raises(IndexError):
        sp.softmax(t, 2)
    with pytest.raises(ValueError):
        sp.softmax(hip_tensor(sp, np.zeros((0, 4), F32)), 1)
    with pytest.raises(ValueError):
        sp.softmax(t.transpose(0, 1))
    with pytest.raises(IndexError):
        sp.log_softmax(t, 5)


# -------------------------------------------------------------- autograd

def run_both(sp, build, arrays):
    """Runs `build(lib, tensors)` on the device and on the oracle; returns the
    losses and leaf gradients of both."""
    dev = [hip_tensor(sp, a, requires_grad=True) for a in arrays]
    ref = [R.RTensor.of(a, requires_grad=True) for a in arrays]
    loss_d = build(sp, dev)
    loss_r = build(R, ref)
    loss_d.backward()
    loss_r.backward()
    return (host(sp, loss_d), loss_r.numpy(), [host(sp, t.grad()) for t in dev],
            [r.grad().numpy() for r in ref])


def weighted_sum(lib, y, weight):
    return lib.sum(lib.multiply(y, weight))


def test_autograd_elementwise_chain_bitexact_grads(sp):
    # loss = sum(((a*b - a/b) + a) * w): gradients pass through elementwise
    # ops and one full sum, whose backward is a broadcast fill (exact).
    a = normal(12, (16, 24))
    b = np.abs(normal(13, (16, 24))) + F32(0.5)
    w = normal(14, (16, 24))

    def build(lib, t):
        y = lib.add(lib.subtract(lib.multiply(t[0], t[1]), lib.divide(t[0], t[1])), t[0])
        return weighted_sum(lib, y, t[2])

    loss_d, loss_r, grads_d, grads_r = run_both(sp, build, [a, b, w])
    assert_red(loss_d, loss_r, a.size, np.sqrt(np.sum(a.astype(np.float64) ** 2)) * 4, "loss")
    for i, (gd, gr) in enumerate(zip(grads_d, grads_r)):
        assert_bitexact(gd, gr, f"grad {i}")


def test_exact_gradient_zero_signs(sp):
    """A gradient that reaches a parent of its own shape is passed on as is by
    default, so a -0.0 element stays -0.0, where the reference adds it into a
    zeroed buffer (tensor.cpp:597-632) and gets +0.0.  With exact zero signs
    on, every gradient equals the oracle's bit for bit, zero signs included:
    d a = 1 * w and d w = 1 * a hold -0.0 where w or a do, and subtract's
    negated gradient turns +0.0 into -0.0."""
    a = normal(40, (8, 16))
    w = normal(41, (8, 16))
    c = normal(43, (8, 16))
    w[0, :4] = -0.0
    w[1, :4] = 0.0
    a[2, :3] = -0.0
    bias = normal(42, (16,))

    def build(lib, t):
        y = lib.subtract(lib.add(lib.multiply(t[0], t[1]), t[2]), lib.multiply(t[3], t[1]))
        return lib.sum(y)

    arrays = [a, w, bias, c]
    assert not sp.exact_gradient_zero_signs()
    _, _, gd, gr = run_both(sp, build, arrays)
    assert np.signbit(gd[0][0, :4]).all() and not np.signbit(gr[0][0, :4]).any()
    sp.set_exact_gradient_zero_signs(True)
    try:
        assert sp.exact_gradient_zero_signs()
        loss_d, loss_r, gd, gr = run_both(sp, build, arrays)
        for i, (got, want) in enumerate(zip(gd, gr)):
            assert_bitexact(got, want, f"grad {i} with exact zero signs")
        # d a = 1 * w and d c = -1 * w at the zeros of w: +0.0 throughout
        for got in (gd[0][:2, :4], gd[3][:2, :4]):
            assert np.all(got == 0) and not np.signbit(got).any()
    finally:
        sp.set_exact_gradient_zero_signs(False)


def test_autograd_unary_chain(sp):
    x = normal(15, (8, 32))
    w = normal(16, (8, 32))
    for name in ["negate", "square", "exp", "sigmoid", "silu", "tanh", "gelu"]:
        def build(lib, t, name=name):
            return weighted_sum(lib, getattr(lib, name)(t[0]), t[1])

        _, _, grads_d, grads_r = run_both(sp, build, [x, w])
        # The backward rules reuse the forward value (y within 2 ulp); rules
        # such as 1 - y*y cancel, so the bound is absolute in |w| as well as
        # relative: |d grad| <= 8 eps (|grad| + |w|).
        eps = np.finfo(F32).eps
        err = np.abs(grads_d[0].astype(np.float64) - grads_r[0])
        assert np.all(err <= 8 * eps * (np.abs(grads_r[0]) + np.abs(w))), f"{name} grad"
        assert_ulp(grads_d[1], grads_r[1], 2, f"{name} weight grad")


def test_autograd_broadcast_reduction_grads(sp):
    # C2 structure at small size: y = x*scale + bias, loss = sum(y*G)
    B, T, Cn = 4, 64, 96
    x = normal(17, (B, T, Cn))
    bias = np.random.default_rng(18).uniform(-0.1, 0.1, Cn).astype(F32)
    scale = np.random.default_rng(19).uniform(0.5, 1.5, (B, 1, Cn)).astype(F32)
    G = normal(20, (B, T, Cn))

    def build(lib, t):
        return weighted_sum(lib, lib.add(lib.multiply(t[0], t[1]), t[2]), t[3])

    _, _, gd, gr = run_both(sp, build, [x, scale, bias, G])
    assert_bitexact(gd[0], gr[0], "dx = G*scale")
    prod = C.binary(G, x, "multiply")
    assert_red(gd[1], gr[1], T, np.sqrt(C.reduce_gradient(prod.astype(np.float64) ** 2, scale.shape)),
               "dscale")
    assert_red(gd[2], gr[2], B * T, np.sqrt(C.reduce_gradient(G.astype(np.float64) ** 2, bias.shape)),
               "dbias")


def test_autograd_reuse_accumulates_in_order(sp):
    # x feeds three ops: contributions accumulate in the engine's order
    x = normal(21, (10, 10))
    w = normal(22, (10, 10))

    def build(lib, t):
        y = lib.add(lib.multiply(t[0], t[0]), lib.multiply_scalar(t[0], 3.0))
        return weighted_sum(lib, y, t[1])

    _, _, gd, gr = run_both(sp, build, [x, w])
    assert_bitexact(gd[0], gr[0], "reused x")


@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("log", [False, True])
def test_autograd_softmax(sp, axis, log):
    x = normal(23, (12, 40), np.sqrt(2))
    w = normal(24, (12, 40))

    def build(lib, t):
        y = lib.log_softmax(t[0], axis) if log else lib.softmax(t[0], axis)
        return weighted_sum(lib, y, t[1])

    _, _, gd, gr = run_both(sp, build, [x, w])
    n = x.shape[axis]
    scale = np.sqrt(np.sum(w.astype(np.float64) ** 2, axis=axis, keepdims=True))
    err = np.abs(gd[0].astype(np.float64) - gr[0])
    assert np.all(err <= 1e-6 * np.sqrt(n) * scale + 8 * np.finfo(F32).eps * (np.abs(gr[0]) + np.abs(w)))


def layer_norm(lib, x, gamma, beta, G):
    # mu = mean(x,1,keepdim); xc = x - mu; var = mean(square(xc),1,keepdim)
    # xhat = xc / sqrt(var + 1e-5); y = xhat*gamma + beta; loss = sum(y*G)
    mu = lib.mean(x, [1], True) if lib is not R else R.mean(x, [1], True)
    xc = lib.subtract(x, mu)
    var = lib.mean(lib.square(xc), [1], True) if lib is not R else R.mean(R.square(xc), [1], True)
    xhat = lib.divide(xc, lib.sqrt(lib.add_scalar(var, 1e-5)))
    y = lib.add(lib.multiply(xhat, gamma), beta)
    return weighted_sum(lib, y, G)


@pytest.mark.parametrize("view", ["transpose", "narrow"])
def test_autograd_layernorm_chain_on_views(sp, view):
    rows, cols = 48, 80
    if view == "transpose":
        base = normal(25, (cols, rows))
    else:
        base = normal(25, (rows + 7, cols + 9))
    gamma = np.random.default_rng(26).uniform(0.5, 1.5, cols).astype(F32)
    beta = np.random.default_rng(27).uniform(-0.1, 0.1, cols).astype(F32)
    G = normal(28, (rows, cols))

    def build(lib, t):
        x = t[0].transpose(0, 1) if view == "transpose" else t[0].narrow(0, 3, rows).narrow(1, 4, cols)
        return layer_norm(lib, x, t[1], t[2], t[3])

    loss_d, loss_r, gd, gr = run_both(sp, build, [base, gamma, beta, G])
    assert_red(loss_d, loss_r, rows * cols, np.sqrt(np.sum(G.astype(np.float64) ** 2)) * 2, "loss")
    # every gradient passes through row means (n = cols) and the final sum
    for i, name in enumerate(["x", "gamma", "beta"]):
        scale = np.max(np.abs(gr[i])) + 1e-30
        err = np.max(np.abs(gd[i].astype(np.float64) - gr[i]))
        assert err <= 1e-6 * np.sqrt(rows * cols) * scale * 8, f"{name}: {err} vs scale {scale}"


@pytest.mark.parametrize("norm", ["layer_norm", "rms_norm"])
@pytest.mark.parametrize("computed", [False, True])
def test_autograd_norm_gradient_written_into_base(sp, norm, computed):
    """A fused norm whose input is a chain of narrows writes that input's
    gradient straight into the gradient of the chain's base, whose border the
    engine zeroes first; the base's gradient is handed down the chain and
    delivered where the chain would have embedded it.  Against the same norm
    on an exact copy of x (x.contiguous() of the strided view, x * 1.0 of the
    contiguous one), whose dense gradient the chain embeds: every
    gradient bit-exact, including the base's second contribution added in
    the same order.  `computed`: the chain starts on base * 2 instead of the
    leaf, so the placed gradient feeds that product's rule."""
    layer = norm == "layer_norm"
    shape = (70, 300) if layer else (70, 256)
    base_np = normal(101, shape)
    rng = np.random.default_rng(102)
    w_np = rng.uniform(0.5, 1.5, 256).astype(F32)
    b_np = rng.uniform(-0.1, 0.1, 256).astype(F32)
    G_np = normal(103, (60, 256))
    H_np = normal(104, shape)

    def run(copy):
        base = hip_tensor(sp, base_np, True)
        w = hip_tensor(sp, w_np, True)
        b = hip_tensor(sp, b_np, True)
        top = sp.multiply_scalar(base, 2.0) if computed else base
        x = top.narrow(0, 5, 60)
        if layer:
            x = x.narrow(1, 20, 256)  # rows 300 apart, read in place
        if copy:  # an exact copy with a node of its own
            x = x.contiguous() if layer else sp.multiply_scalar(x, 1.0)
        y = sp.layer_norm(x, w, b, 1e-5) if layer else sp.rms_norm(x, w, 1e-5)
        loss = sp.add(weighted_sum(sp, y, hip_tensor(sp, G_np)),
                      weighted_sum(sp, base, hip_tensor(sp, H_np)))
        before = sp.autograd_counters()
        loss.backward()
        after = sp.autograd_counters()
        grads = [host(sp, base.grad()), host(sp, w.grad())] + ([host(sp, b.grad())] if layer else [])
        return grads, after["placed_gradients"] - before["placed_gradients"]

    placed, count = run(copy=False)
    embedded, count_copy = run(copy=True)
    assert count == 1 and count_copy == 0
    for got, want, name in zip(placed, embedded, ["base", "weight", "bias"]):
        assert_bitexact(got, want, f"{norm} {name}")
    box = (slice(5, 65), slice(20, 276)) if layer else (slice(5, 65), slice(None))
    outside = np.ones(shape, bool)
    outside[box] = False
    # outside the box the first term's gradient is zero (through the product
    # too), so only the second term's remains
    assert_bitexact(placed[0][outside], H_np[outside], "border holds only the second term")


def test_autograd_narrow_chains_embed_once(sp):
    """A chain of narrows is embedded into its base once: each narrow whose
    input is a narrow with no other consumer hands its gradient down with
    the composed box.  The gradients are bit-exact against the oracle, which
    embeds one narrow at a time; an intermediate view with a second consumer
    breaks the chain there, and a chain that ends on a computed tensor
    embeds into it before that op's rule runs."""
    base = normal(91, (13, 17, 9))
    G = normal(92, (5, 10, 6))
    H = normal(93, (8, 17, 9))

    def chain(t):
        return t.narrow(0, 2, 8).narrow(2, 1, 6).narrow(1, 3, 10).narrow(0, 1, 5)

    def build(lib, t):
        return weighted_sum(lib, chain(t[0]), t[1])

    before = sp.autograd_counters()
    loss_d, loss_r, gd, gr = run_both(sp, build, [base, G])
    after = sp.autograd_counters()
    assert after["window_fusions"] == before["window_fusions"] + 3
    assert_bitexact(gd[0], gr[0], "base through four narrows")
    want = np.zeros_like(base)
    want[3:8, 3:13, 1:7] = G  # every element of G times the ones of the sum
    assert_bitexact(gd[0], want, "embedded box")

    # v = base.narrow(0, 2, 8) also feeds a second product: the chain stops
    # above v, which adds the two gradients before its own embedding
    def build_shared(lib, t):
        v = t[0].narrow(0, 2, 8)
        first = weighted_sum(lib, v.narrow(1, 3, 10).narrow(2, 1, 6), t[1])
        return lib.add(first, weighted_sum(lib, v, t[2]))

    G8 = normal(94, (8, 10, 6))
    before = sp.autograd_counters()
    _, _, gd, gr = run_both(sp, build_shared, [base, G8, H])
    after = sp.autograd_counters()
    assert after["window_fusions"] == before["window_fusions"] + 1
    assert_bitexact(gd[0], gr[0], "base with a shared intermediate view")

    # the chain ends on a product, not a leaf
    def build_computed(lib, t):
        u = lib.multiply_scalar(t[0], 3.0)
        return weighted_sum(lib, u.narrow(1, 2, 12).narrow(0, 4, 6), t[1])

    G6 = normal(95, (6, 12, 9))
    _, _, gd, gr = run_both(sp, build_computed, [base, G6])
    assert_bitexact(gd[0], gr[0], "base through a product and two narrows")


GRAPH_SHAPE = (6, 8, 8)
GRAPH_LEAVES = [(10, 12, 11), GRAPH_SHAPE, (8, 9, 8)]


def random_graph(seed, steps=24):
    """A random recipe over three leaves: view chains (narrow, transpose)
    from the larger leaves down to GRAPH_SHAPE, scaled copies of whole
    leaves that are then narrowed (a chain that ends on a computed tensor),
    views shared by several chains, and exact elementwise arithmetic
    (add, subtract, multiply, divide by 1 + y*y, negate, square, scalar
    scale and shift) on GRAPH_SHAPE nodes, with tensors reused by several
    consumers.  Unary and scalar ops take contiguous tensors only, as in
    the reference (unary.cpp, elementwise.cpp), so they are applied to
    leaves and computed nodes, never to views.  Every node that nothing
    consumes is summed into the loss, so every leaf reaches it.  Returns
    the recipe and the sink nodes.

    Magnitudes are followed with float32 numpy values: a node above 64 is
    scaled by 1/256 (an exact power of two) before it is used further."""
    rng = np.random.default_rng(seed)
    values = [normal(seed * 10 + k, s) for k, s in enumerate(GRAPH_LEAVES)]
    shapes = [tuple(s) for s in GRAPH_LEAVES]
    consumed = [False] * len(shapes)
    dense = [True] * len(shapes)  # leaves and computed nodes are contiguous
    recipe = []

    def emit(step, value):
        for i in step[1:]:
            if isinstance(i, tuple):  # node references are tagged ("n", index)
                consumed[i[1]] = True
        recipe.append(step)
        values.append(value.astype(F32))
        shapes.append(tuple(value.shape))
        consumed.append(False)
        dense.append(step[0] not in ("narrow", "transpose"))
        node = len(values) - 1
        if np.max(np.abs(values[node])) > 64:
            return emit(("scale", ("n", node), 1.0 / 256.0), values[node] * F32(1.0 / 256.0))
        return node

    def view_step(i):
        shape = shapes[i]
        narrowable = [a for a in range(3) if shape[a] > GRAPH_SHAPE[a]]
        if rng.random() < 0.2 and shape[1] >= 8 and shape[2] >= 8:
            return emit(("transpose", ("n", i)), np.swapaxes(values[i], 1, 2))
        axis = int(rng.choice(narrowable))
        length = int(rng.integers(GRAPH_SHAPE[axis], shape[axis]))
        start = int(rng.integers(0, shape[axis] - length + 1))
        index = [slice(None)] * 3
        index[axis] = slice(start, start + length)
        return emit(("narrow", ("n", i), axis, start, length), values[i][tuple(index)])

    def chain_to_shape(i):
        while shapes[i] != GRAPH_SHAPE:
            i = view_step(i)
        return i

    for leaf in (0, 2):
        chain_to_shape(leaf)
    for _ in range(steps):
        pick = rng.random()
        ready = [i for i, s in enumerate(shapes) if s == GRAPH_SHAPE]
        large = [i for i, s in enumerate(shapes) if s != GRAPH_SHAPE]
        if pick < 0.25 and large:
            i = int(rng.choice(large))
            if rng.random() < 0.3 and i in (0, 2):
                c = float(rng.choice([0.5, -2.0, 3.0]))
                i = emit(("scale", ("n", i), c), values[i] * F32(c))
            chain_to_shape(view_step(i) if shapes[i] != GRAPH_SHAPE else i)
        elif pick < 0.5 and any(dense[i] for i in ready):
            i = int(rng.choice([i for i in ready if dense[i]]))
            kind = str(rng.choice(["negate", "square", "scale", "shift"]))
            if kind == "negate":
                emit(("negate", ("n", i)), -values[i])
            elif kind == "square":
                emit(("square", ("n", i)), values[i] * values[i])
            elif kind == "scale":
                c = float(rng.choice([0.75, -1.5, 2.0]))
                emit(("scale", ("n", i), c), values[i] * F32(c))
            else:
                c = float(rng.choice([0.25, -1.0]))
                emit(("shift", ("n", i), c), values[i] + F32(c))
        else:
            i, j = (int(k) for k in rng.choice(ready, 2))
            kind = str(rng.choice(["add", "subtract", "multiply", "divide"]))
            if kind == "divide":
                square = ("square", ("n", j)) if dense[j] else ("multiply", ("n", j), ("n", j))
                sq = emit(square, values[j] * values[j])
                j = emit(("shift", ("n", sq), 1.0), values[sq] + F32(1.0))
            op = {"add": np.add, "subtract": np.subtract, "multiply": np.multiply,
                  "divide": np.divide}[kind]
            emit((kind, ("n", i), ("n", j)), op(values[i], values[j]))
    sinks = [i for i, s in enumerate(shapes) if s == GRAPH_SHAPE and not consumed[i]]
    return recipe, sinks


def replay_graph(lib, leaves, recipe, sinks):
    """Builds the recipe on `lib` and returns the sum of its sinks."""
    nodes = list(leaves)
    for step in recipe:
        kind = step[0]
        x = nodes[step[1][1]]
        if kind == "narrow":
            nodes.append(x.narrow(step[2], step[3], step[4]))
        elif kind == "transpose":
            nodes.append(x.transpose(1, 2))
        elif kind == "scale":
            nodes.append(lib.multiply_scalar(x, step[2]))
        elif kind == "shift":
            nodes.append(lib.add_scalar(x, step[2]))
        elif kind in ("negate", "square"):
            nodes.append(getattr(lib, kind)(x))
        else:
            nodes.append(getattr(lib, kind)(x, nodes[step[2][1]]))
    total = nodes[sinks[0]]
    for i in sinks[1:]:
        total = lib.add(total, nodes[i])
    return total


@pytest.mark.parametrize("exact_signs", [False, True])
def test_random_autograd_graphs(sp, exact_signs):
    """Sixteen random graphs (random_graph) run through the engine and
    through the oracle's engine, which follows autograd.cpp:201-265 one
    node at a time.  Every op on the way is exact IEEE arithmetic or a
    view, so the leaf gradients agree bit for bit when exact zero signs
    are on, and in value (+0 and -0 taken as equal) by default; the loss
    is a full sum, compared with its red bound.  The graphs exercise the
    engine's narrow-chain hand-down, gradients placed into a base, shared
    intermediate views, chains that end on a computed tensor and the
    accumulation order of reused tensors."""
    sp.set_exact_gradient_zero_signs(exact_signs)
    before = sp.autograd_counters()["window_fusions"]
    try:
        for seed in range(300, 316):
            recipe, sinks = random_graph(seed)
            arrays = [normal(seed * 10 + k, s) for k, s in enumerate(GRAPH_LEAVES)]
            arrays.append(normal(seed * 10 + 7, GRAPH_SHAPE))

            def build(lib, t, recipe=recipe, sinks=sinks):
                return weighted_sum(lib, replay_graph(lib, t[:3], recipe, sinks), t[3])

            loss_d, loss_r, gd, gr = run_both(sp, build, arrays)
            total = replay_graph(R, [R.RTensor.of(a) for a in arrays[:3]], recipe, sinks).numpy()
            terms = total.astype(np.float64) * arrays[3]
            assert_red(loss_d, loss_r, terms.size, np.sqrt(np.sum(terms ** 2)), f"seed {seed} loss")
            for k, (got, want) in enumerate(zip(gd, gr)):
                what = f"seed {seed} ({len(recipe)} steps) grad {k}"
                if exact_signs:
                    assert_bitexact(got, want, what)
                else:
                    assert_bitexact(got + F32(0), want + F32(0), what)
        assert sp.autograd_counters()["window_fusions"] > before, "no narrow chain was handed down"
    finally:
        sp.set_exact_gradient_zero_signs(False)


def test_autograd_api_errors(sp):
    x = hip_tensor(sp, normal(1, (3,)), requires_grad=True)
    y = sp.multiply(x, x)
    with pytest.raises(ValueError):
        y.backward()  # not one element
    loss = sp.sum(y)
    loss.backward()
    g1 = host(sp, x.grad())
    sp.sum(sp.multiply(x, x)).backward()
    assert_bitexact(host(sp, x.grad()), g1 + g1, "second backward accumulates")
    x.zero_grad()
    assert not x.has_grad
    with pytest.raises(ValueError):
        y.grad()
    with pytest.raises(ValueError):
        hip_tensor(sp, np.arange(3, dtype=np.int64)).set_requires_grad(True)


def test_autograd_view_gradients_are_dense(sp):
    """Leaf gradients are dense, as the reference's clones made them
    (autograd.cpp:145, :244): through a transpose a leaf's gradient is
    contiguous, adds into it across backward calls pair the right elements,
    an identity that receives a gradient through a view and one directly
    adds them elementwise, and AdamW accepts the gradient of a Parameter
    used through a transpose."""
    x = normal(81, (3, 4))
    c = normal(82, (4, 3))
    d = normal(83, (3, 4))

    def build(lib, t):
        through_view = lib.sum(lib.multiply(t[0].transpose(0, 1), t[1]))
        direct = lib.sum(lib.multiply(t[0], t[2]))
        return lib.add(through_view, direct)

    dev = [hip_tensor(sp, a, requires_grad=True) for a in (x, c, d)]
    ref = [R.RTensor.of(a, requires_grad=True) for a in (x, c, d)]
    for _ in range(2):  # two backward calls accumulate into the leaves
        build(sp, dev).backward()
        build(R, ref).backward()
    got = dev[0].grad()
    assert got.is_contiguous()
    assert_bitexact(host(sp, got), ref[0].grad().numpy(), "x grad, two calls")
    assert_bitexact(host(sp, dev[1].grad()), ref[1].grad().numpy(), "c grad")

    # a Parameter used only through a transpose: AdamW takes its gradient
    w = sp.nn.Parameter(hip_tensor(sp, x))
    opt = sp.optim.AdamW([w], 1e-3)
    sp.sum(sp.multiply(w.tensor().transpose(0, 1), hip_tensor(sp, c))).backward()
    assert w.grad().is_contiguous()
    assert_bitexact(host(sp, w.grad()), c.T.copy(), "parameter grad through a transpose")
    opt.step()


def memory_stats():
    import ctypes

    from spar_amd import hip

    stats = hip.MemoryStats()
    hip.call("spar_hip_memory_stats", ctypes.byref(stats), 0)
    return stats


def test_layernorm_chain_second_run_allocates_nothing_and_copies_no_gradient(sp):
    """A C5-shaped LayerNorm chain on a transposed view, forward and backward,
    twice: the second run takes every block from the caching allocator (no
    hipMalloc, cache hits > 0), and the engine copies no leaf gradient
    (transpose's backward already returns a contiguous gradient; the
    reference cloned every contribution, autograd.cpp:145, :244).  It adds
    one pair out of place: x's gradient from subtract and the stride-0
    broadcast view that mean's backward returns, read in place instead of
    filled out; the other pairs add in place."""
    device = sp.Device.hip(0)
    rng = np.random.default_rng(71)
    base = sp.Tensor.from_numpy(rng.standard_normal((2048, 1024)).astype(np.float32)).to(device)
    gamma = sp.Tensor.from_numpy(rng.uniform(0.5, 1.5, 2048).astype(np.float32)).to(device)
    beta = sp.Tensor.from_numpy(rng.uniform(-0.1, 0.1, 2048).astype(np.float32)).to(device)
    G = sp.Tensor.from_numpy(rng.standard_normal((1024, 2048)).astype(np.float32)).to(device)
    for leaf in (base, gamma, beta):
        leaf.set_requires_grad(True)

    def run():
        for leaf in (base, gamma, beta):
            leaf.zero_grad()
        x = base.transpose(0, 1)
        mu = sp.mean(x, [1], True)
        xc = sp.subtract(x, mu)
        var = sp.mean(sp.square(xc), [1], True)
        y = sp.add(sp.multiply(sp.divide(xc, sp.sqrt(sp.add_scalar(var, 1e-5))), gamma), beta)
        sp.sum(sp.multiply(y, G), None, False).backward()
        sp.synchronize(device)
        return [leaf.grad().to(sp.Device.cpu()).numpy() for leaf in (base, gamma, beta)]

    first = run()
    stats_before = memory_stats()
    counters_before = sp.autograd_counters()
    second = run()
    stats_after = memory_stats()
    counters_after = sp.autograd_counters()
    assert stats_after.device_allocations == stats_before.device_allocations
    assert stats_after.cache_hits > stats_before.cache_hits
    assert counters_after["backward_calls"] == counters_before["backward_calls"] + 1
    assert counters_after["leaf_copies"] == counters_before["leaf_copies"]
    assert counters_after["out_of_place_adds"] == counters_before["out_of_place_adds"] + 1
    # x feeds mean and subtract, xc feeds square and divide: in-place adds
    assert counters_after["in_place_adds"] > counters_before["in_place_adds"]
    for a, b in zip(first, second):
        assert_bitexact(b, a, "second run")
