"""AdamW, gradient scaling and the gradient-norm summary on the GPU against
the oracle's restatement of Spar's CPU loops (optim/adamw.cpp:37-61,
training/gradients.cpp:28-111), through the C ABI and through the
nn / training / optim API.

Tolerances: AdamW and scaling are bit-exact (the same IEEE double operations
in the same order, rounded to the parameter dtype as the CPU loop does).  The
norm summary's `scale` (the largest finite magnitude) and its flags are
exact; `scaled_sum_squares` and the norm are sums of squares evaluated in
another order than the CPU loop, both in double, so they carry red(N) in
double precision: relative error <= 64 * sqrt(N) * 2^-53, far below one
float32 ulp of any gradient element.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle.ops as O
import oracle.reference as R
from tests.helpers import assert_bitexact

pytestmark = pytest.mark.gpu

F32, F64 = np.float32, np.float64


def norm_tolerance(count):
    return 64 * math.sqrt(max(count, 1)) * 2.0 ** -53


class Placed:
    """A device copy of a 1-D array at `offset` elements past a 256-byte
    aligned block (offset 1 makes every pointer misaligned for 16 bytes)."""

    def __init__(self, hip, array, offset=0):
        self.hip = hip
        self.array = np.ascontiguousarray(array)
        self.offset = offset * self.array.itemsize
        self.buffer = hip.DeviceBuffer(self.array.nbytes + self.offset + 16)
        if self.array.nbytes:
            hip.call("spar_hip_copy_host_to_device", self.ptr, self.array.ctypes.data,
                     self.array.nbytes, 0)

    @property
    def ptr(self):
        return self.buffer.address(self.offset)

    def numpy(self):
        out = np.empty_like(self.array)
        if out.nbytes:
            self.hip.call("spar_hip_copy_device_to_host", out.ctypes.data, self.ptr, out.nbytes, 0)
        return out


def adamw_abi(hip, p, g, m, v, hyper, step, offset=0):
    lr, b1, b2, eps, wd = hyper
    dev = [Placed(hip, a, offset) for a in (p, g, m, v)]
    hip.call("spar_hip_launch_adamw", dev[0].ptr, dev[1].ptr, dev[2].ptr, dev[3].ptr, p.size,
             hip.dtype_tag(p.dtype), lr, b1, b2, eps, wd, O.adamw_correction(b1, step),
             O.adamw_correction(b2, step), 0)
    return dev[0].numpy(), dev[2].numpy(), dev[3].numpy()


HYPER = [(1e-3, 0.9, 0.999, 1e-8, 0.01), (0.3, 0.5, 0.7, 1e-3, 0.5), (0.0, 0.0, 0.0, 1.0, 0.0)]


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("hyper", HYPER)
def test_adamw_bitexact(hip, dtype, hyper):
    rng = np.random.default_rng(100)
    for n, offset in [(1, 0), (3, 0), (4, 0), (5, 1), (1023, 0), (4099, 1), (1 << 20 | 7, 0)]:
        p = rng.standard_normal(n).astype(dtype)
        m = np.zeros(n, dtype)
        v = np.zeros(n, dtype)
        for step in (1, 2, 3):
            g = (rng.standard_normal(n) * 10.0 ** rng.integers(-4, 4, n)).astype(dtype)
            gp, gm, gv = adamw_abi(hip, p, g, m, v, hyper, step, offset)
            O.adamw(p, g, m, v, *hyper, O.adamw_correction(hyper[1], step),
                    O.adamw_correction(hyper[2], step))
            what = f"n={n} offset={offset} step={step} {np.dtype(dtype).name} {hyper}"
            assert_bitexact(gm, m, "first moment " + what)
            assert_bitexact(gv, v, "second moment " + what)
            assert_bitexact(gp, p, "parameter " + what)


@pytest.mark.parametrize("dtype", [F32, F64])
def test_adamw_special_values(hip, dtype):
    info = np.finfo(dtype)
    g = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, info.max, -info.max, info.tiny,
                  info.smallest_subnormal, -info.smallest_subnormal, 1e-30, 1e30], dtype)
    n = g.size
    p = np.array([1.0, -1.0, 2.0, -2.0, 0.0, -0.0, info.max, -info.max, np.inf, np.nan,
                  info.smallest_subnormal, 3.0], dtype)
    m = np.linspace(-1, 1, n).astype(dtype)
    v = np.abs(np.linspace(-2, 1, n)).astype(dtype)
    for hyper in HYPER[:2]:
        for step in (1, 7):
            got = adamw_abi(hip, p, g, m, v, hyper, step)
            want = [a.copy() for a in (p, m, v)]
            O.adamw(want[0], g, want[1], want[2], *hyper, O.adamw_correction(hyper[1], step),
                    O.adamw_correction(hyper[2], step))
            for name, a, b in zip(("parameter", "first", "second"), got, want):
                assert_bitexact(a, b, f"{name} {np.dtype(dtype).name} {hyper} step {step}")


def test_adamw_argument_checks(hip):
    lib = hip.load()
    assert lib.spar_hip_launch_adamw(None, None, None, None, 0, hip.FLOAT32, 1e-3, 0.9, 0.999,
                                     1e-8, 0.0, 0.1, 0.001, 0).code == 0
    assert lib.spar_hip_launch_adamw(None, None, None, None, 4, hip.FLOAT32, 1e-3, 0.9, 0.999,
                                     1e-8, 0.0, 0.1, 0.001, 0).code == 1
    assert lib.spar_hip_launch_adamw(None, None, None, None, 0, hip.INT32, 1e-3, 0.9, 0.999,
                                     1e-8, 0.0, 0.1, 0.001, 0).code == 1


@pytest.mark.parametrize("dtype", [F32, F64])
def test_scale_in_place_bitexact(hip, dtype):
    rng = np.random.default_rng(101)
    for n, offset in [(1, 0), (7, 1), (4096, 0), (100003, 1)]:
        x = (rng.standard_normal(n) * 10.0 ** rng.integers(-30, 30, n)).astype(dtype)
        x[:3] = [np.nan, np.inf, -0.0][: min(3, n)]
        for factor in (0.1, 1.0 / 3.0, 1e-300, 1e300, 0.0, -2.5):
            dev = Placed(hip, x, offset)
            hip.call("spar_hip_launch_scale_in_place", dev.ptr, n, hip.dtype_tag(dtype), factor, 0)
            want = x.copy()
            O.scale(want, factor)
            assert_bitexact(dev.numpy(), want, f"n={n} offset={offset} factor={factor}")
    lib = hip.load()
    assert lib.spar_hip_launch_scale_in_place(None, 0, hip.FLOAT32, math.inf, 0).code == 1
    assert lib.spar_hip_launch_scale_in_place(None, 0, hip.FLOAT32, 2.0, 0).code == 0


def summary_of(hip, x, offset=0):
    dev = Placed(hip, x, offset)
    summary = hip.NormSummary()
    hip.call("spar_hip_gradient_norm_summary", ctypes.byref(summary), dev.ptr, x.size,
             hip.dtype_tag(x.dtype), 0)
    return summary


def check_summary(summary, x, what):
    want = O.SumSquares().add(x)
    assert summary.has_infinity == int(want.has_infinity), f"{what}: infinity flag"
    assert summary.has_nan == int(want.has_nan), f"{what}: NaN flag"
    assert summary.scale == want.scale, f"{what}: scale {summary.scale} != {want.scale}"
    tol = norm_tolerance(x.size)
    assert abs(summary.scaled_sum_squares - want.scaled_sum_squares) <= \
        tol * want.scaled_sum_squares, f"{what}: scaled sum of squares"
    got_norm = O.SumSquares().combine(summary.scale, summary.scaled_sum_squares,
                                      summary.has_infinity, summary.has_nan).norm()
    want_norm = want.norm()
    if math.isnan(want_norm):
        assert math.isnan(got_norm), what
    elif math.isinf(want_norm) or want_norm == 0.0:
        assert got_norm == want_norm, what
    else:
        assert abs(got_norm - want_norm) <= tol * want_norm, f"{what}: norm"


@pytest.mark.parametrize("dtype", [F32, F64])
def test_norm_summary_matches_oracle(hip, dtype):
    rng = np.random.default_rng(102)
    for n, offset in [(1, 0), (2, 1), (5, 0), (63, 1), (4096, 0), (65537, 1), (1_000_003, 0),
                      (1 << 24, 0)]:
        x = (rng.standard_normal(n) * 10.0 ** rng.integers(-6, 6, n)).astype(dtype)
        check_summary(summary_of(hip, x, offset), x, f"n={n} offset={offset}")


def test_norm_summary_float64_range(hip):
    """Squares that overflow or underflow double, and mixed extremes."""
    rng = np.random.default_rng(103)
    for scale in (1e300, 1e-300, 1e-310):
        x = rng.standard_normal(100000) * scale
        check_summary(summary_of(hip, x), x, f"scale {scale}")
    x = rng.standard_normal(100000) * 10.0 ** rng.integers(-300, 300, 100000)
    check_summary(summary_of(hip, x), x, "mixed extremes")
    x = np.full(4097, np.finfo(F64).max)
    check_summary(summary_of(hip, x), x, "all DBL_MAX")
    x = np.full(4097, np.finfo(F32).max, F32)
    check_summary(summary_of(hip, x), x, "all FLT_MAX")


@pytest.mark.parametrize("dtype", [F32, F64])
def test_norm_summary_special_values(hip, dtype):
    rng = np.random.default_rng(104)
    n = 300007
    for positions, values in [([0], [np.nan]), ([n // 2], [np.inf]), ([n - 1], [-np.inf]),
                              ([5, n - 2], [np.inf, np.nan]), ([], [])]:
        x = rng.standard_normal(n).astype(dtype)
        x[positions] = values
        check_summary(summary_of(hip, x), x, f"{np.dtype(dtype).name} {positions}")
    for x in (np.zeros(1000, dtype), np.array([-0.0], dtype), np.array([np.nan] * 9, dtype),
              np.array([np.inf, 0.0], dtype),
              np.full(1000, np.finfo(dtype).smallest_subnormal, dtype)):
        check_summary(summary_of(hip, x), x, f"{x[:3]}")
    empty = hip.NormSummary(7.0, 7.0, 7, 7)
    hip.call("spar_hip_gradient_norm_summary", ctypes.byref(empty), None, 0, hip.FLOAT32, 0)
    assert (empty.scale, empty.scaled_sum_squares, empty.has_infinity, empty.has_nan) == \
        (0.0, 1.0, 0, 0)


def test_norm_summary_device_form(hip):
    """The device-memory form writes the same summary as the host form."""
    rng = np.random.default_rng(105)
    xs = [rng.standard_normal(n).astype(F32) for n in (0, 1, 4096, 123457)]
    xs.append(np.array([1.0, np.nan], F32))
    size = ctypes.sizeof(hip.NormSummary)
    out = hip.DeviceBuffer(size * len(xs))
    devs = [Placed(hip, x) for x in xs]
    for k, (x, d) in enumerate(zip(xs, devs)):
        hip.call("spar_hip_launch_gradient_norm_summary", out.address(k * size), d.ptr, x.size,
                 hip.FLOAT32, 0)
    raw = (hip.NormSummary * len(xs))()
    hip.call("spar_hip_copy_device_to_host", ctypes.addressof(raw), out.ptr, size * len(xs), 0)
    for k, x in enumerate(xs):
        host = summary_of(hip, x)
        got = raw[k]
        assert (got.scale, got.scaled_sum_squares, got.has_infinity, got.has_nan) == \
            (host.scale, host.scaled_sum_squares, host.has_infinity, host.has_nan), k


# ---------------------------------------------------------------- the API

@pytest.fixture(scope="module")
def sp():
    from spar_amd import spar

    if spar.hip_device_count() < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    return spar


def parameters_with_gradients(sp, arrays, weights, dtype=F32):
    """Parameters on hip:0 with gradients from sum(p * w) (gradient = w)."""
    device = sp.Device.hip(0)
    params = [sp.nn.Parameter(sp.Tensor.from_numpy(a.astype(dtype)).to(device)) for a in arrays]
    for param, w in zip(params, weights):
        if w is not None:
            sp.sum(sp.multiply(param.tensor(), sp.Tensor.from_numpy(w.astype(dtype)).to(device))).backward()
    return params


def host(sp, tensor):
    return tensor.to(sp.Device.cpu()).numpy()


@pytest.mark.parametrize("dtype", [F32, F64])
def test_adamw_api_matches_oracle(sp, dtype):
    rng = np.random.default_rng(106)
    shapes = [(64, 33), (1000,), (3, 5, 7)]
    arrays = [rng.standard_normal(s).astype(dtype) for s in shapes]
    params = parameters_with_gradients(sp, arrays, [None] * 3, dtype)
    params.append(params[0])  # a duplicate identity is tracked once
    opt = sp.optim.AdamW(params, learning_rate=1e-2, weight_decay=0.05)
    assert opt.parameter_count() == 3
    ref = R.AdamW([a.copy() for a in arrays], 1e-2, 0.9, 0.999, 1e-8, 0.05)
    device = sp.Device.hip(0)
    for step in range(4):
        grads = []
        for k, param in enumerate(params[:3]):
            param.zero_grad()
            if step == 1 and k == 2:  # a Parameter without a gradient is skipped
                grads.append(None)
                continue
            w = (rng.standard_normal(shapes[k]) * 10.0 ** (k - 1)).astype(dtype)
            sp.sum(sp.multiply(param.tensor(), sp.Tensor.from_numpy(w).to(device))).backward()
            grads.append(host(sp, param.grad()))
        opt.step()
        ref.step(grads)
        for k, param in enumerate(params[:3]):
            assert_bitexact(host(sp, param.tensor()), ref.parameters[k], f"step {step} param {k}")
    state = opt.parameter_state(params[2])
    assert state.step == 3
    assert_bitexact(host(sp, state.first_moment), ref.states[2][0], "first moment")
    assert_bitexact(host(sp, state.second_moment), ref.states[2][1], "second moment")


def test_adamw_api_state_and_errors(sp):
    device = sp.Device.hip(0)
    p = sp.nn.Parameter(sp.Tensor.from_numpy(np.ones(4, F32)).to(device))
    other = sp.nn.Parameter(sp.Tensor.from_numpy(np.ones(4, F32)).to(device))
    opt = sp.optim.AdamW([p])
    assert opt.tracks(p) and not opt.tracks(other) and not opt.tracks(p.clone())
    assert opt.parameter_state(p) is None
    with pytest.raises(ValueError, match="does not track"):
        opt.parameter_state(other)
    zeros = sp.Tensor.from_numpy(np.zeros(4, F32)).to(device)
    with pytest.raises(ValueError, match="at least one"):
        opt.set_parameter_state(p, sp.optim.AdamWParameterState(zeros, zeros, 0))
    with pytest.raises(ValueError, match="mismatch"):
        opt.set_parameter_state(p, sp.optim.AdamWParameterState(zeros, zeros.to(sp.Device.cpu()), 2))
    m = sp.Tensor.from_numpy(np.full(4, 0.5, F32)).to(device)
    v = sp.Tensor.from_numpy(np.full(4, 0.25, F32)).to(device)
    opt.set_parameter_state(p, sp.optim.AdamWParameterState(m, v, 5))
    g = np.array([1.0, -2.0, 0.5, 0.0], F32)
    sp.sum(sp.multiply(p.tensor(), sp.Tensor.from_numpy(g).to(device))).backward()
    opt.step()
    want_p, want_m, want_v = np.ones(4, F32), np.full(4, 0.5, F32), np.full(4, 0.25, F32)
    O.adamw(want_p, g, want_m, want_v, 1e-3, 0.9, 0.999, 1e-8, 0.01,
            O.adamw_correction(0.9, 6), O.adamw_correction(0.999, 6))
    assert_bitexact(host(sp, p.tensor()), want_p, "restored state step")
    assert opt.parameter_state(p).step == 6
    opt.zero_grad()
    assert not p.has_grad()
    for kwargs, message in [({"learning_rate": -1.0}, "learning_rate"), ({"beta1": 1.0}, "beta1"),
                            ({"beta2": math.nan}, "beta2"), ({"epsilon": 0.0}, "epsilon"),
                            ({"weight_decay": -0.1}, "weight_decay")]:
        with pytest.raises(ValueError, match=message):
            sp.optim.AdamW([p], **kwargs)
    with pytest.raises(ValueError, match="learning_rate"):
        opt.set_learning_rate(math.inf)
    with pytest.raises(ValueError, match="floating-point"):
        sp.nn.Parameter(sp.Tensor.from_numpy(np.ones(3, np.int32)).to(device))


def test_global_norm_and_clip_api(sp):
    rng = np.random.default_rng(107)
    arrays = [rng.standard_normal(s).astype(F32) for s in [(300, 17), (5,), (4096,), (2, 2)]]
    weights = [rng.standard_normal(a.shape).astype(F32) * 3 for a in arrays]
    weights[3] = None  # no gradient: not active
    params = parameters_with_gradients(sp, arrays, weights)
    params.append(params[1])  # duplicates count once
    grads = [None if w is None else w.copy() for w in weights]
    want = R.global_grad_norm(grads)
    got = sp.training.global_grad_norm(params)
    assert abs(got - want) <= norm_tolerance(sum(a.size for a in arrays)) * want
    result = sp.training.clip_grad_norm(params, 2 * want)
    assert not result.clipped and result.scale == 1.0 and result.total_norm == got
    result = sp.training.clip_grad_norm(params, 1.5)
    assert result.clipped and result.scale == 1.5 / result.total_norm
    R.scale_gradients(grads, result.scale)
    for k in range(3):
        assert_bitexact(host(sp, params[k].grad()), grads[k], f"clipped gradient {k}")
    sp.training.scale_gradients(params, 0.5)
    R.scale_gradients(grads, 0.5)
    for k in range(3):
        assert_bitexact(host(sp, params[k].grad()), grads[k], f"scaled gradient {k}")
    assert sp.training.global_grad_norm([]) == 0.0
    assert sp.training.global_grad_norm(params[3:4]) == 0.0
    with pytest.raises(ValueError, match="finite and nonnegative"):
        sp.training.clip_grad_norm(params, -1.0)
    with pytest.raises(ValueError, match="finite"):
        sp.training.scale_gradients(params, math.nan)


def test_clip_rejects_nonfinite_before_scaling(sp):
    arrays = [np.ones(8, F32), np.ones(8, F32)]
    weights = [np.full(8, 2.0, F32), np.array([1, 2, np.inf, 4, 5, 6, 7, 8], F32)]
    params = parameters_with_gradients(sp, arrays, weights)
    assert sp.training.global_grad_norm(params) == math.inf
    with pytest.raises(RuntimeError, match="nonfinite"):
        sp.training.clip_grad_norm(params, 1.0)
    assert_bitexact(host(sp, params[0].grad()), weights[0], "untouched after the error")
    weights[1][0] = np.nan
    params = parameters_with_gradients(sp, arrays, weights)
    assert math.isnan(sp.training.global_grad_norm(params))


def test_parameter_move_to_keeps_identity(sp):
    """nn.move_to (parameter.cpp:54-87): values move between the host and
    hip:0 in place; aliases, earlier Tensor handles and the autograd identity
    follow; a live gradient refuses the move and changes nothing."""
    rng = np.random.default_rng(108)
    cpu, device = sp.Device.cpu(), sp.Device.hip(0)
    values = rng.standard_normal((33, 5)).astype(F32)
    p = sp.nn.Parameter(sp.Tensor.from_numpy(values))
    tracked = sp.optim.AdamW([p])  # holds a C++ copy of the Parameter
    handle = p.tensor()
    assert handle.device == cpu
    sp.nn.move_to([p, p], device)  # duplicates move once
    assert p.tensor().device == device and handle.device == device
    assert tracked.tracks(p)
    assert_bitexact(host(sp, p.tensor()), values, "values after the move")
    w = rng.standard_normal((33, 5)).astype(F32)
    sp.sum(sp.multiply(p.tensor(), sp.Tensor.from_numpy(w).to(device))).backward()
    assert p.has_grad()
    with pytest.raises(sp.LogicError, match="live gradient"):
        sp.nn.move_to([p], cpu)
    assert p.tensor().device == device  # unchanged by the refused move
    assert_bitexact(host(sp, p.grad()), w, "gradient after the refused move")
    p.zero_grad()
    sp.nn.move_to([p], cpu)
    assert p.tensor().device == cpu and handle.device == cpu
    assert_bitexact(p.tensor().numpy(), values, "values back on the host")
    sp.nn.move_to([p], cpu)  # already there: nothing to do


@pytest.mark.parametrize("dtype", [F32, F64])
def test_adamw_move_to_round_trip_is_bitexact(sp, dtype):
    """AdamW.move_to: moments and Parameters go to the host and back; the
    steps after the round trip equal those of an optimizer that never moved."""
    rng = np.random.default_rng(109)
    cpu, device = sp.Device.cpu(), sp.Device.hip(0)
    shapes = [(40, 7), (129,)]
    arrays = [rng.standard_normal(s).astype(dtype) for s in shapes]
    grads = [[rng.standard_normal(s).astype(dtype) for s in shapes] for _ in range(3)]

    def run(move):
        params = [sp.nn.Parameter(sp.Tensor.from_numpy(a).to(device)) for a in arrays]
        opt = sp.optim.AdamW(params, learning_rate=3e-3, weight_decay=0.1)
        for step in range(3):
            for param, g in zip(params, grads[step]):
                param.zero_grad()
                sp.sum(sp.multiply(param.tensor(), sp.Tensor.from_numpy(g).to(device))).backward()
            opt.step()
            if move and step == 1:
                opt.zero_grad()
                opt.move_to(cpu)
                for param in params:
                    assert param.tensor().device == cpu
                    state = opt.parameter_state(param)
                    assert state.first_moment.device == cpu and state.second_moment.device == cpu
                opt.move_to(device)
        return [host(sp, p.tensor()) for p in params], [opt.parameter_state(p) for p in params]

    moved, moved_states = run(True)
    still, still_states = run(False)
    for k in range(len(shapes)):
        assert_bitexact(moved[k], still[k], f"parameter {k}")
        assert moved_states[k].step == still_states[k].step == 3
        assert_bitexact(host(sp, moved_states[k].first_moment), host(sp, still_states[k].first_moment),
                        f"first moment {k}")
        assert_bitexact(host(sp, moved_states[k].second_moment),
                        host(sp, still_states[k].second_moment), f"second moment {k}")


def test_adamw_move_to_refused_with_gradients(sp):
    device = sp.Device.hip(0)
    p = sp.nn.Parameter(sp.Tensor.from_numpy(np.ones(6, F32)).to(device))
    opt = sp.optim.AdamW([p])
    sp.sum(sp.multiply(p.tensor(), p.tensor())).backward()
    opt.step()
    with pytest.raises(sp.LogicError, match="live gradient"):
        opt.move_to(sp.Device.cpu())
    state = opt.parameter_state(p)
    assert state.first_moment.device == device  # nothing committed


def test_adamw_full_size_step(hip):
    """One AdamW step over GPT-2 small's 124,439,808 fp32 parameters, bit-exact,
    and the gradient norm over the same gradient within red(N)."""
    n = 124_439_808
    rng = np.random.default_rng(108)
    p = rng.standard_normal(n, dtype=F32)
    g = rng.standard_normal(n, dtype=F32) * F32(1e-2)
    m = rng.standard_normal(n, dtype=F32) * F32(1e-3)
    v = np.abs(rng.standard_normal(n, dtype=F32)) * F32(1e-5)
    hyper = (3e-4, 0.9, 0.95, 1e-8, 0.1)
    got = adamw_abi(hip, p, g, m, v, hyper, 1000)
    O.adamw(p, g, m, v, *hyper, O.adamw_correction(0.9, 1000), O.adamw_correction(0.95, 1000))
    assert_bitexact(got[0], p, "parameter")
    assert_bitexact(got[1], m, "first moment")
    assert_bitexact(got[2], v, "second moment")
    check_summary(summary_of(hip, g), g, "full-size gradient")
