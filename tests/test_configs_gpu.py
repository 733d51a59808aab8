"""Parity at the benchmark configurations' full sizes (C1-C5).

Inputs come from the device generators with the benchmark's seeds and are
copied back for the oracle, so both sides see the same bytes.  Where the
oracle finishes in seconds at full size it checks every element; otherwise it
checks sampled rows, and size-independent properties cover the whole output:
probability rows sum to one, log-sum-exp of log-probabilities is zero,
checksums of checksums agree, argmax points at the maximum, and gradients
with a closed form (d beta = column sums of G) match it.
"""
import numpy as np
import pytest

from oracle import ops as ref
from tests.helpers import assert_bitexact, assert_red, assert_ulp
from tests.test_kernels_gpu import (log_softmax_tolerance_check, softmax_backward_bound,
                                    softmax_tolerance_check)

pytestmark = pytest.mark.gpu

F32 = np.float32


def normal(hip, n, seed, std=1.0):
    buffer = hip.DeviceBuffer(n * 4)
    hip.call("spar_hip_random_normal", buffer.ptr, n, hip.FLOAT32, seed, 0.0, std, 0)
    return buffer


def uniform(hip, n, seed, low, high):
    buffer = hip.DeviceBuffer(n * 4)
    hip.call("spar_hip_random_uniform", buffer.ptr, n, hip.FLOAT32, seed, low, high, 0)
    return buffer


def host(buffer, shape, dtype=F32):
    return buffer.to_numpy(dtype, shape)


def norm2(a, axis=None, keepdims=False):
    return np.sqrt(np.sum(np.square(a, dtype=np.float64), axis=axis, keepdims=keepdims))


def sample_rows(count, total, seed):
    rows = np.random.default_rng(seed).choice(total, size=count, replace=False)
    return np.sort(np.concatenate([[0, total - 1], rows]))


def red_mean(terms, axis):
    """The RED bound (1e-6 sqrt(n) times the larger of |sum| and the terms'
    2-norm) of an n-term sum along `axis`, divided by n: the bound on a mean
    computed by any summation order."""
    n = terms.shape[axis]
    total = np.sum(terms, axis=axis, keepdims=True)
    return 1e-6 * np.sqrt(n) * np.maximum(np.abs(total), norm2(terms, axis=axis, keepdims=True)) / n


def layernorm_bounds(x, gamma, beta, G, eps_norm=1e-5):
    """First-order bounds on how far two float32 LayerNorm implementations
    whose row statistics each lie within RED of the exact ones can disagree,
    forward and backward, from the float64 values of the chain's quantities:

      mu = mean(x), var = mean(xc^2), sd = sqrt(var + eps), xhat = xc / sd,
      y = xhat gamma + beta, g = G gamma, A = mean(g), B = mean(g xhat),
      dx = (g - A - xhat B) / sd, d gamma = sum_rows G xhat, d beta = sum_rows G.

    Each side's error in mu, var, A and B is at most red_mean of its terms
    (B also carries the propagated error of xhat); xhat moves by
    d_mu / sd + |xhat| d_sd / sd with d_sd = d_var / (2 sd); each quantity
    is bounded by the sum of |partial derivative| x error over the
    statistics it depends on, doubled for the two sides, plus 8 eps of the
    magnitudes of its terms for the roundings of its own operations."""
    eps = float(np.finfo(F32).eps)
    x64 = x.astype(np.float64)
    rows = x64.shape[0]
    mu = x64.mean(axis=1, keepdims=True)
    xc = x64 - mu
    var = (xc * xc).mean(axis=1, keepdims=True)
    sd = np.sqrt(var + eps_norm)
    xhat = xc / sd
    d_mu = red_mean(x64, 1)
    d_sd = red_mean(xc * xc, 1) / (2 * sd)
    d_xhat = d_mu / sd + np.abs(xhat) * d_sd / sd
    g = G.astype(np.float64) * gamma
    A = g.mean(axis=1, keepdims=True)
    B = (g * xhat).mean(axis=1, keepdims=True)
    dx = (g - A - xhat * B) / sd
    d_A = red_mean(g, 1)
    d_B = red_mean(g * xhat, 1) + np.mean(np.abs(g) * d_xhat, axis=1, keepdims=True)
    y = xhat * gamma + beta
    bound_y = 2 * np.abs(gamma) * d_xhat + 8 * eps * (np.abs(y) + np.abs(xhat * gamma) + np.abs(beta))
    bound_dx = (2 * (d_A + np.abs(xhat) * d_B + d_xhat * np.abs(B) + np.abs(dx) * d_sd)
                + 8 * eps * (np.abs(g) + np.abs(A) + np.abs(xhat * B) + np.abs(dx) * sd)) / sd
    gx = G.astype(np.float64) * xhat
    bound_dgamma = (2 * rows * red_mean(gx, 0)[0] + 2 * np.sum(np.abs(G) * d_xhat, axis=0)
                    + 8 * eps * np.abs(gx.sum(axis=0)))
    bound_dbeta = 2 * rows * red_mean(G.astype(np.float64), 0)[0]
    tiny = float(np.finfo(F32).tiny)
    return bound_y + tiny, bound_dx + tiny, bound_dgamma + tiny, bound_dbeta + tiny


def assert_within(got, want, bound, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ok = err <= bound
    assert ok.all(), (f"{what}: {int((~ok).sum())} outside the derived bound, worst excess "
                      f"{np.max(err - bound):.3e} (bound there {bound.ravel()[np.argmax(err - bound)]:.3e})")


# ------------------------------------------------------------------ C1

def test_c1_contiguous_elementwise(hip):
    shape = (4096, 4096)
    n = shape[0] * shape[1]
    a, b, out = normal(hip, n, 1), normal(hip, n, 2), hip.DeviceBuffer(n * 4)
    ha, hb = host(a, shape), host(b, shape)
    for name, op in (("add", hip.ADD), ("multiply", hip.MULTIPLY)):
        hip.call("spar_hip_launch_binary", out.ptr, a.ptr, b.ptr, n, hip.FLOAT32, op, 0)
        assert_bitexact(host(out, shape), ref.binary(ha, hb, name), f"C1 {name}")
    assert np.abs(ha).max() <= 10.0  # exp(clip(a, -10, 10)) is exp(a) on this draw
    for name, op in (("exp", hip.EXP), ("gelu", hip.GELU)):
        hip.call("spar_hip_launch_unary", out.ptr, a.ptr, n, hip.FLOAT32, op, 0)
        assert_ulp(host(out, shape), ref.unary(ha, name), 2, f"C1 {name}")


# ------------------------------------------------------------------ C2

def test_c2_broadcast_forward_and_backward(hip):
    B, T, C = 32, 1024, 4096
    n = B * T * C
    u = hip.u64_array
    x, G = normal(hip, n, 11), normal(hip, n, 14)
    bias, scale = uniform(hip, C, 12, -0.1, 0.1), uniform(hip, B * C, 13, 0.5, 1.5)
    hx, hG = host(x, (B, T, C)), host(G, (B, T, C))
    hbias, hscale = host(bias, (C,)), host(scale, (B, 1, C))
    y = hip.DeviceBuffer(n * 4)
    shape, dense = u([B, T, C]), u([T * C, C, 1])

    hip.call("spar_hip_launch_strided_binary", y.ptr, x.ptr, dense, 0, bias.ptr, u([0, 0, 1]), 0,
             3, shape, hip.FLOAT32, hip.ADD, 0)
    assert_bitexact(host(y, (B, T, C)), ref.binary(hx, hbias, "add"), "x + bias")
    hip.call("spar_hip_launch_strided_binary", y.ptr, x.ptr, dense, 0, scale.ptr, u([C, 0, 1]), 0,
             3, shape, hip.FLOAT32, hip.MULTIPLY, 0)
    assert_bitexact(host(y, (B, T, C)), ref.binary(hx, hscale, "multiply"), "x * scale")
    hip.call("spar_hip_launch_strided_binary", y.ptr, G.ptr, dense, 0, scale.ptr, u([C, 0, 1]), 0,
             3, shape, hip.FLOAT32, hip.MULTIPLY, 0)
    assert_bitexact(host(y, (B, T, C)), ref.binary(hG, hscale, "multiply"), "dx = G * scale")

    # d bias = sum over (B, T) of G: every column against the oracle, and the
    # checksum of checksums against the full sum of G
    dbias = hip.DeviceBuffer(C * 4)
    hip.call("spar_hip_launch_broadcast_reduce", dbias.ptr, G.ptr, 3, shape, 1, u([C]),
             u([0] * 8), n, hip.FLOAT32, 0)
    got = host(dbias, (C,))
    assert_red(got, ref.reduce_gradient(hG, (C,)), B * T, norm2(hG, axis=(0, 1)), "d bias")
    assert_red(np.sum(got, dtype=np.float64), ref.full_reduce(hG, "sum"), n, norm2(hG),
               "sum of d bias vs sum of G")

    # d scale = sum over T of G * x (fused), against multiply-then-reduce
    dscale = hip.DeviceBuffer(B * C * 4)
    hip.call("spar_hip_launch_multiply_reduce", dscale.ptr, G.ptr, x.ptr, 3, shape, 3,
             u([B, 1, C]), n, hip.FLOAT32, 0)
    product = ref.binary(hG, hx, "multiply")
    assert_red(host(dscale, (B, 1, C)), ref.reduce_gradient(product, (B, 1, C)), T,
               norm2(product, axis=1, keepdims=True), "d scale")


# ------------------------------------------------------------------ C3

def test_c3_axis_and_full_reductions(hip):
    R = 8192
    n = R * R
    x = normal(hip, n, 3)
    hx = host(x, (R, R))
    u = hip.u64_array
    out = hip.DeviceBuffer(R * 8)
    sums = {}
    for axis in (1, 0):
        kept = 1 - axis

        def run(code, dtype=F32):
            hip.call("spar_hip_launch_axis_reduction", out.ptr, x.ptr, 2, u([R, R]), u([R, 1]), 0,
                     1 << axis, hip.FLOAT32, code, 0)
            return host(out, (R,), dtype)

        norm = norm2(hx, axis=axis)
        want_sum = ref.axis_sum(hx, [axis])
        sums[axis] = run(hip.SUM)
        assert_red(sums[axis], want_sum, R, norm, f"sum axis {axis}")
        assert_red(run(hip.MEAN), ref.scalar(want_sum, "divide", float(R)), R, norm / R,
                   f"mean axis {axis}")
        want_max, want_arg = ref.axis_max(hx, [axis])
        got_max, got_arg = run(hip.MAX), run(hip.ARGMAX, np.int64)
        assert_bitexact(got_max, want_max, f"max axis {axis}")
        assert_bitexact(got_arg, want_arg, f"argmax axis {axis}")
        picked = hx[got_arg, np.arange(R)] if axis == 0 else hx[np.arange(R), got_arg]
        assert np.array_equal(picked, got_max), f"x[argmax] == max, axis {axis} (kept {kept})"
    total = ref.full_reduce(hx, "sum")
    for axis in (0, 1):
        assert_red(np.sum(sums[axis], dtype=np.float64), total, n, norm2(hx),
                   f"checksum of axis-{axis} sums")

    n = 1 << 28
    v = uniform(hip, n, 4, -1.0, 1.0)
    hv = host(v, (n,))
    scalar_out = hip.DeviceBuffer(8)
    norm = norm2(hv)
    for kind, code in (("sum", hip.SUM), ("mean", hip.MEAN)):
        hip.call("spar_hip_launch_reduction", scalar_out.ptr, v.ptr, n, hip.FLOAT32, code, 0)
        assert_red(host(scalar_out, (1,))[0], ref.full_reduce(hv, kind), n,
                   norm / (n if kind == "mean" else 1), f"full {kind} 2^28")
    hip.call("spar_hip_launch_reduction", scalar_out.ptr, v.ptr, n, hip.FLOAT32, hip.MAX, 0)
    assert host(scalar_out, (1,))[0] == ref.full_reduce(hv, "max"), "full max 2^28"


# ------------------------------------------------------------------ C4

@pytest.mark.parametrize("log", [False, True])
def test_c4_softmax_rows(hip, log):
    rows, V = 8192, 32768
    n = rows * V
    logits, G = normal(hip, n, 5, np.sqrt(2.0)), normal(hip, n, 6)
    out, dx = hip.DeviceBuffer(n * 4), hip.DeviceBuffer(n * 4)
    undefined = hip.DeviceBuffer(rows * 4)
    hip.call("spar_hip_launch_probability_forward", out.ptr, undefined.ptr, logits.ptr, rows, V, 1,
             hip.FLOAT32, int(log), 0)
    hip.call("spar_hip_launch_probability_backward", dx.ptr, G.ptr, out.ptr, undefined.ptr, rows,
             V, 1, hip.FLOAT32, int(log), 0)
    hl, hG = host(logits, (rows, V)), host(G, (rows, V))
    hy, hdx = host(out, (rows, V)), host(dx, (rows, V))
    assert not host(undefined, (rows,), np.int32).any(), "no C4 row is undefined"

    # every row: probabilities sum to one / log-sum-exp is zero
    eps = np.finfo(F32).eps
    if log:
        lse = np.log(np.sum(np.exp(hy.astype(np.float64)), axis=1))
        assert np.all(np.abs(lse) <= 1e-6 * np.sqrt(V) + 8 * eps), "log-sum-exp of rows"
    else:
        assert np.all(hy >= 0)
        row_sums = np.sum(hy, axis=1, dtype=np.float64)
        assert np.all(np.abs(row_sums - 1.0) <= 1e-6 * np.sqrt(V) + 8 * eps), "rows sum to one"

    # every row against the oracle, forward and backward, in blocks of 512
    # rows (the oracle's C loops take about 20 s for all 8192 on one core)
    for first in range(0, rows, 512):
        block = slice(first, first + 512)
        sub, gsub = hl[block], hG[block]
        what = f"C4 rows {first}-{first + 511}"
        if log:
            want, flags = ref.log_softmax(sub, 1)
            log_softmax_tolerance_check(hy[block], want, V, F32, what + " log_softmax")
            want_dx = ref.log_softmax_backward(gsub, hy[block], flags, 1)
        else:
            want, flags = ref.softmax_axis(sub, 1)
            softmax_tolerance_check(hy[block], want, V, F32, what + " softmax")
            want_dx = ref.softmax_axis_backward(gsub, hy[block], flags, 1)
        assert not flags.any(), what + ": the oracle marks no row undefined"
        bound = softmax_backward_bound(gsub, hy[block], V, F32, log)
        err = np.abs(hdx[block].astype(np.float64) - want_dx)
        assert np.all(err <= bound), f"{what} backward: max excess {np.max(err - bound)}"


# ------------------------------------------------------------------ C5

@pytest.mark.parametrize("view", ["transposed", "sliced"])
def test_c5_layernorm_chain(hip, view):
    """The LayerNorm chain of the benchmark through the Tensor API, forward
    and backward, on a [4096, 8192] view.  Rows are independent in the
    forward and in d x, so sampled rows are checked against the oracle run on
    those rows; d beta has the closed form sum over rows of G; d gamma is the
    sum over rows of G * xhat (checked against float64)."""
    from spar_amd import spar

    import oracle.reference as R

    rows, cols = 4096, 8192
    device = spar.Device.hip(0)
    rng = np.random.default_rng(60 if view == "transposed" else 61)
    if view == "transposed":
        base = rng.standard_normal((cols, rows)).astype(F32)
    else:
        base = rng.standard_normal((4608, 9216)).astype(F32)
    gamma = rng.uniform(0.5, 1.5, cols).astype(F32)
    beta = rng.uniform(-0.1, 0.1, cols).astype(F32)
    G = rng.standard_normal((rows, cols)).astype(F32)

    def view_of(lib_tensor, is_ref):
        if view == "transposed":
            return lib_tensor.transpose(0, 1)
        return lib_tensor.narrow(0, 256, rows).narrow(1, 512, cols)

    def chain(lib, x, g, b, w):
        mu = lib.mean(x, [1], True)
        xc = lib.subtract(x, mu)
        var = lib.mean(lib.square(xc), [1], True)
        xhat = lib.divide(xc, lib.sqrt(lib.add_scalar(var, 1e-5)))
        y = lib.add(lib.multiply(xhat, g), b)
        return xhat, y, lib.sum(lib.multiply(y, w), None, False)

    tensors = []
    for array in (base, gamma, beta, G):
        t = spar.Tensor.from_numpy(array).to(device)
        t.set_requires_grad(True)
        tensors.append(t)
    xhat, y, loss = chain(spar, view_of(tensors[0], False), tensors[1], tensors[2], tensors[3])
    loss.backward()
    cpu = spar.Device.cpu()
    got_xhat, got_y = xhat.to(cpu).numpy(), y.to(cpu).numpy()
    got_dbase = tensors[0].grad().to(cpu).numpy()
    got_dgamma, got_dbeta = tensors[1].grad().to(cpu).numpy(), tensors[2].grad().to(cpu).numpy()
    got_dx = got_dbase.T if view == "transposed" else got_dbase[256:256 + rows, 512:512 + cols]
    if view == "sliced":
        outside = got_dbase.copy()
        outside[256:256 + rows, 512:512 + cols] = 0
        assert not outside.any(), "gradient outside the slice is zero"

    # Every row against the chain evaluated in float64 on the host, then
    # sampled rows against the oracle's restatement (the reference's float32
    # operations and order).  Bound: 1e-6 * sqrt(n) of the row's largest
    # magnitude; the oracle's own float32 chain stays within 0.02 of that
    # bound of the float64 values on these inputs.
    x_host = base.T if view == "transposed" else base[256:256 + rows, 512:512 + cols]
    x64 = x_host.astype(np.float64)
    xc64 = x64 - x64.mean(axis=1, keepdims=True)
    sd64 = np.sqrt((xc64 * xc64).mean(axis=1, keepdims=True) + 1e-5)
    xhat64 = xc64 / sd64
    y64 = xhat64 * gamma + beta
    g64 = G.astype(np.float64) * gamma
    dx64 = (g64 - g64.mean(axis=1, keepdims=True)
            - xhat64 * (g64 * xhat64).mean(axis=1, keepdims=True)) / sd64
    tol = 1e-6 * np.sqrt(cols)
    for name, got, want in (("xhat", got_xhat, xhat64), ("y", got_y, y64), ("dx", got_dx, dx64)):
        scale = np.max(np.abs(want), axis=1, keepdims=True) + 1e-30
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= tol * scale), f"C5 {view} {name} vs float64: max rel {np.max(err / scale)}"

    picked = sample_rows(128, rows, 62)
    sub = [R.RTensor.of(np.ascontiguousarray(x_host[picked]), requires_grad=True),
           R.RTensor.of(gamma, requires_grad=True), R.RTensor.of(beta, requires_grad=True),
           R.RTensor.of(np.ascontiguousarray(G[picked]))]
    want_xhat, want_y, want_loss = chain(R, sub[0], sub[1], sub[2], sub[3])
    want_loss.backward()
    for name, got, want in (("xhat", got_xhat[picked], want_xhat.numpy()),
                            ("y", got_y[picked], want_y.numpy()),
                            ("dx", got_dx[picked], sub[0].grad().numpy())):
        scale = np.max(np.abs(want), axis=1, keepdims=True) + 1e-30
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= tol * scale), f"C5 {view} {name} vs oracle: max rel {np.max(err / scale)}"

    # d beta = sum over rows of G (closed form); d gamma = sum over rows of
    # G * xhat with xhat from the host's float64 chain
    assert_red(got_dbeta, ref.axis_sum(G, [0]), rows, norm2(G, axis=0), "d beta")
    # d gamma against float64: its own sum within red(rows), plus the row
    # statistics' error carried by xhat (one side of layernorm_bounds'
    # two-implementation bound)
    want_dgamma = np.sum(G.astype(np.float64) * xhat64, axis=0)
    assert_within(got_dgamma, want_dgamma, layernorm_bounds(x_host, gamma, beta, G)[2] / 2,
                  f"C5 {view} d gamma vs float64")


@pytest.mark.parametrize("view", ["transposed", "sliced"])
def test_c5_fused_layernorm_matches_chain(hip, view):
    """The fused LayerNorm on the C5 views against the composed chain
    (validated against the oracle above), forward and backward, at full size:
    the transposed view takes the column-layout passes, the block of a wider
    base the row kernels and one embedding of the two narrows' gradient."""
    from spar_amd import spar

    rows, cols = 4096, 8192
    device, cpu = spar.Device.hip(0), spar.Device.cpu()
    rng = np.random.default_rng(63)
    if view == "transposed":
        base = rng.standard_normal((cols, rows)).astype(F32)
    else:
        base = rng.standard_normal((rows + 512, cols + 1024)).astype(F32)
    gamma = rng.uniform(0.5, 1.5, cols).astype(F32)
    beta = rng.uniform(-0.1, 0.1, cols).astype(F32)
    G = rng.standard_normal((rows, cols)).astype(F32)

    def run(fused):
        ts = []
        for array in (base, gamma, beta, G):
            t = spar.Tensor.from_numpy(array).to(device)
            t.set_requires_grad(True)
            ts.append(t)
        x = (ts[0].transpose(0, 1) if view == "transposed"
             else ts[0].narrow(0, 256, rows).narrow(1, 512, cols))
        if fused:
            y = spar.layer_norm(x, ts[1], ts[2], 1e-5)
        else:
            mu = spar.mean(x, [1], True)
            xc = spar.subtract(x, mu)
            sd = spar.sqrt(spar.add_scalar(spar.mean(spar.square(xc), [1], True), 1e-5))
            y = spar.add(spar.multiply(spar.divide(xc, sd), ts[1]), ts[2])
        spar.sum(spar.multiply(y, ts[3]), None, False).backward()
        return [y.to(cpu).numpy()] + [t.grad().to(cpu).numpy() for t in ts[:3]]

    fused, chain = run(True), run(False)
    if view == "transposed":
        x_rows, dx_fused, dx_chain = base.T, fused[1].T, chain[1].T
    else:
        x_rows = base[256:256 + rows, 512:512 + cols]
        dx_fused = fused[1][256:256 + rows, 512:512 + cols]
        dx_chain = chain[1][256:256 + rows, 512:512 + cols]
        outside = np.ones(base.shape, bool)
        outside[256:256 + rows, 512:512 + cols] = False
        assert not fused[1][outside].any(), "gradient outside the block"
    bound_y, bound_dx, bound_dgamma, bound_dbeta = layernorm_bounds(x_rows, gamma, beta, G)
    assert_within(fused[0], chain[0], bound_y, f"C5 {view} fused y")
    assert_within(dx_fused, dx_chain, bound_dx, f"C5 {view} fused dx")
    assert_within(fused[2], chain[2], bound_dgamma, f"C5 {view} fused d gamma")
    assert_within(fused[3], chain[3], bound_dbeta, f"C5 {view} fused d beta")
