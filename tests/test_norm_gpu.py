"""Fused LayerNorm / RMSNorm against the oracle's composition of the
reference's ops (RMSNorm::forward, nn/rmsnorm.cpp:50-52; LayerNorm is the
same chain with centring and a bias).

The fused kernels compute every element with the composed path's float
operations; only the order of the two row sums differs (a tree instead of a
sequential scan).  Each row statistic therefore differs by at most red(n)
(relative 1e-6 sqrt(n) at the row's natural scale), and every output element
of the row moves by that relative amount of the row's magnitude, plus a few
roundings.  The bounds below are those, with the row's largest output as the
scale -- for dx, the largest term of the difference it is, since
dx = (g w - mean(g w) - xhat mean(g w xhat)) / d cancels (entirely so for a
one-element RMSNorm row, where xhat^2 is nearly 1).
"""
import numpy as np
import pytest

import oracle.reference as R
from oracle import ops as ref
from tests.helpers import assert_bitexact, assert_red

pytestmark = pytest.mark.gpu

F32, F64 = np.float32, np.float64
EPSILON = 1.0e-5


def tag(dtype):
    return 0 if np.dtype(dtype) == F32 else 1


_alive = []


@pytest.fixture(autouse=True)
def _release_buffers():
    yield
    _alive.clear()


def dev(hip, array):
    buffer = hip.DeviceBuffer.from_numpy(np.ascontiguousarray(array))
    _alive.append(buffer)
    return buffer


def out_buf(hip, count, dtype):
    buffer = hip.DeviceBuffer(max(count, 1) * np.dtype(dtype).itemsize)
    _alive.append(buffer)
    return buffer


def data(rows, n, dtype, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, n)) * 2 + 0.5).astype(dtype)
    w = rng.uniform(0.5, 1.5, n).astype(dtype)
    b = rng.uniform(-0.1, 0.1, n).astype(dtype)
    g = rng.standard_normal((rows, n)).astype(dtype)
    return x, w, b, g


def composed_forward(x, w, b, center):
    """The composed chain through the oracle's op loops: (y, mu, d)."""
    n = x.shape[1]
    mu = None
    xc = x
    if center:
        mu = ref.scalar(ref.axis_sum(x, [1]), "divide", float(n))
        xc = ref.binary(x, mu[:, None], "subtract")
    var = ref.scalar(ref.axis_sum(ref.unary(xc, "square"), [1]), "divide", float(n))
    d = ref.unary(ref.scalar(var, "add", EPSILON), "sqrt")
    y = ref.binary(ref.binary(xc, d[:, None], "divide"), w, "multiply")
    if center:
        y = ref.binary(y, b, "add")
    return y, mu, d


def row_bound(want, n, dtype, factor=8.0, terms=None):
    """factor * 1e-6 sqrt(n) + 8 eps of the row's scale: its largest |value|,
    or, where the value is a difference of larger terms (dx), the largest
    term of that difference."""
    scale = np.max(np.abs(want.astype(np.float64)), axis=-1, keepdims=True)
    if terms is not None:
        scale = np.maximum(scale, np.max(terms, axis=-1, keepdims=True))
    return (factor * 1e-6 * np.sqrt(n) + 8 * np.finfo(dtype).eps) * scale + np.finfo(dtype).tiny


def assert_rows(got, want, n, dtype, what, factor=8.0, terms=None):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = row_bound(want, n, dtype, factor, terms)
    assert np.all(err <= bound), f"{what}: worst excess {np.max(err - bound)}"


def dx_terms(g, w, x, center):
    """|g w| / d per element: the size of the terms dx = (g w - ...) / d
    subtracts (float64 statistics)."""
    x64 = x.astype(np.float64)
    xc = x64 - x64.mean(axis=-1, keepdims=True) if center else x64
    d = np.sqrt(np.mean(xc * xc, axis=-1, keepdims=True) + EPSILON)
    return np.abs(g.astype(np.float64) * w.astype(np.float64)) / d


def shapes(dtype):
    limit = 16384 if dtype == F32 else 8192
    return [(5, 1), (3, 3), (7, 8), (64, 100), (9, 1000), (4, 1030), (33, 4096), (6, 8192),
            (3, limit), (2, limit - 4), (3, limit - 1)]


def forward_device(hip, x, w, b, center, dtype):
    rows, n = x.shape
    y, mu, d = out_buf(hip, rows * n, dtype), out_buf(hip, rows, dtype), out_buf(hip, rows, dtype)
    dx = dev(hip, x)
    hip.call("spar_hip_launch_norm_forward", y.ptr, mu.ptr if center else None, d.ptr, dx.ptr, n, 1,
             dev(hip, w).ptr, dev(hip, b).ptr if center else None, rows, n, EPSILON, int(center),
             tag(dtype), 0)
    return (y.to_numpy(dtype, (rows, n)), mu.to_numpy(dtype, (rows,)) if center else None,
            d.to_numpy(dtype, (rows,)), (dx, mu, d))


def test_max_extent(hip):
    lib = hip.load()
    assert lib.spar_hip_norm_max_extent(0) == 16384
    assert lib.spar_hip_norm_max_extent(1) == 8192
    assert lib.spar_hip_norm_max_extent(2) == 0


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("center", [True, False])
def test_norm_forward_kernel(hip, dtype, center):
    for index, (rows, n) in enumerate(shapes(dtype)):
        x, w, b, _ = data(rows, n, dtype, 100 + index)
        got_y, got_mu, got_d, _ = forward_device(hip, x, w, b, center, dtype)
        want_y, want_mu, want_d = composed_forward(x, w, b, center)
        what = f"{'layer' if center else 'rms'} norm {rows}x{n} {np.dtype(dtype).name}"
        if center:
            assert_red(got_mu, want_mu, n, np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=1)) / n,
                       what + " mean")
        assert np.all(np.abs(got_d.astype(np.float64) - want_d) <=
                      (4e-6 * np.sqrt(n) + 4 * np.finfo(dtype).eps) * want_d), what + " d"
        assert_rows(got_y, want_y, n, dtype, what + " y")


@pytest.mark.parametrize("center", [True, False])
def test_norm_forward_rows_beyond_one_grid(hip, center):
    """More rows than one launch grid holds (2^20): the rows go out in
    several grids, each with its own row offset into y, mu and d."""
    rows, n = (1 << 20) + 7, 4
    x, w, b, _ = data(rows, n, F32, 300)
    got_y, got_mu, got_d, _ = forward_device(hip, x, w, b, center, F32)
    want_y, want_mu, want_d = composed_forward(x, w, b, center)
    what = f"{'layer' if center else 'rms'} norm {rows}x{n}"
    if center:
        assert_red(got_mu, want_mu, n, np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=1)) / n,
                   what + " mean")
    assert np.all(np.abs(got_d.astype(np.float64) - want_d) <=
                  (4e-6 * np.sqrt(n) + 4 * np.finfo(F32).eps) * want_d), what + " d"
    assert_rows(got_y, want_y, n, F32, what + " y")


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("center", [True, False])
def test_norm_backward_kernel(hip, dtype, center):
    for index, (rows, n) in enumerate(shapes(dtype)[:-2] + [(300, 64), (1000, 12)]):
        x, w, b, g = data(rows, n, dtype, 200 + index)
        _, _, _, (dx_in, mu, d) = forward_device(hip, x, w, b, center, dtype)
        dx, dw, db = out_buf(hip, rows * n, dtype), out_buf(hip, n, dtype), out_buf(hip, n, dtype)
        hip.call("spar_hip_launch_norm_backward", dx.ptr, n, dw.ptr, db.ptr if center else None,
                 dev(hip, g).ptr, dx_in.ptr, n, 1, dev(hip, w).ptr, mu.ptr if center else None,
                 d.ptr, rows, n, int(center), tag(dtype), 0)
        tx = R.RTensor.of(x, requires_grad=True)
        tw = R.RTensor.of(w, requires_grad=True)
        tb = R.RTensor.of(b, requires_grad=True)
        y = R.layer_norm(tx, tw, tb, EPSILON) if center else R.rms_norm(tx, tw, EPSILON)
        R.sum(R.multiply(y, R.RTensor.of(g))).backward()
        what = f"{'layer' if center else 'rms'} norm backward {rows}x{n} {np.dtype(dtype).name}"
        assert_rows(dx.to_numpy(dtype, (rows, n)), tx.grad().numpy(), n, dtype, what + " dx", 16.0,
                    dx_terms(g, w, x, center))
        # d weight = sum over rows of g * xhat: red(rows) plus each term's
        # relative perturbation through xhat
        _, _, want_d = composed_forward(x, w, b, center)
        xc = x.astype(np.float64) - (x.astype(np.float64).mean(axis=1, keepdims=True) if center else 0)
        terms = np.abs(g.astype(np.float64) * xc / want_d[:, None])
        norm = np.sqrt(np.sum(terms ** 2, axis=0))
        slack = 8e-6 * np.sqrt(n) * np.sum(terms, axis=0)
        err = np.abs(dw.to_numpy(dtype, (n,)).astype(np.float64) - tw.grad().numpy())
        bound = 1e-6 * np.sqrt(rows) * np.maximum(np.abs(tw.grad().numpy()), norm) + slack + 1e-30
        assert np.all(err <= bound), f"{what} d weight: worst excess {np.max(err - bound)}"
        if center:
            assert_red(db.to_numpy(dtype, (n,)), tb.grad().numpy(), rows,
                       np.sqrt(np.sum(g.astype(np.float64) ** 2, axis=0)), what + " d bias")


def test_norm_entry_points_reject_bad_arguments(hip):
    lib = hip.load()
    p = out_buf(hip, 64, F32).ptr
    bad = [
        (p, p, p, p, 8, 1, p, p, 4, 0, EPSILON, 1, 0, 0),            # extent 0
        (p, p, p, p, 16385, 1, p, p, 4, 16385, EPSILON, 1, 0, 0),    # beyond the float32 limit
        (p, p, p, p, 8193, 1, p, p, 4, 8193, EPSILON, 1, 1, 0),      # beyond the float64 limit
        (p, None, p, p, 8, 1, p, p, 4, 8, EPSILON, 1, 0, 0),         # LayerNorm without mean
        (p, p, p, p, 8, 1, p, None, 4, 8, EPSILON, 1, 0, 0),         # LayerNorm without bias
        (p, p, p, p, 8, 1, p, p, 4, 8, EPSILON, 2, 0, 0),            # center flag
        (p, p, p, p, 8, 1, p, p, 4, 8, EPSILON, 1, 2, 0),            # integer dtype
        (p, p, p, p, 8, 1, p, p, 4, 8, -1.0, 1, 0, 0),               # negative epsilon
        (p, p, p, p, 7, 1, p, p, 4, 8, EPSILON, 1, 0, 0),            # rows overlap
        (p, p, p, p, 1, 3, p, p, 4, 8, EPSILON, 1, 0, 0),            # columns overlap
        (p, p, p, p, 8, 2, p, p, 4, 8, EPSILON, 1, 0, 0),            # neither layout
    ]
    for args in bad:
        assert lib.spar_hip_launch_norm_forward(*args).code == 1, args
    backward_bad = [
        (p, 8, p, None, p, p, 8, 1, p, p, p, 4, 8, 1, 0, 0),  # LayerNorm without a bias gradient
        (p, 8, p, p, p, p, 6, 1, p, p, p, 4, 8, 1, 0, 0),     # rows overlap
        (p, 8, p, p, p, p, 1, 3, p, p, p, 4, 8, 1, 0, 0),     # columns overlap
        (p, 8, p, p, p, p, 8, 2, p, p, p, 4, 8, 1, 0, 0),     # neither layout
        (p, 7, p, p, p, p, 8, 1, p, p, p, 4, 8, 1, 0, 0),     # dx rows overlap
        (p, 3, p, p, p, p, 1, 4, p, p, p, 4, 8, 1, 0, 0),     # dx columns overlap
    ]
    for args in backward_bad:
        assert lib.spar_hip_launch_norm_backward(*args).code == 1, args
    # zero rows: parameter gradients are zero, nothing else is touched
    dw, db = out_buf(hip, 8, F32), out_buf(hip, 8, F32)
    hip.call("spar_hip_launch_norm_backward", None, 8, dw.ptr, db.ptr, None, None, 8, 1, p, None,
             None, 0, 8, 1, 0, 0)
    assert not dw.to_numpy(F32, (8,)).any() and not db.to_numpy(F32, (8,)).any()


# ------------------------------------------------------------------ API

@pytest.fixture(scope="module")
def sp():
    from spar_amd import spar

    if spar.hip_device_count() < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    return spar


def api_both(sp, arrays, build):
    device = sp.Device.hip(0)
    on_device = []
    for a in arrays:
        t = sp.Tensor.from_numpy(np.ascontiguousarray(a)).to(device)
        t.set_requires_grad(True)
        on_device.append(t)
    on_oracle = [R.RTensor.of(a, requires_grad=True) for a in arrays]
    yd, yr = build(sp, on_device), build(R, on_oracle)
    cpu = sp.Device.cpu()
    got_y = yd.to(cpu).numpy()
    want_y = yr.numpy()
    return got_y, want_y, on_device, on_oracle


def test_rms_norm_rejects_views_like_the_composition(sp):
    # RMSNorm::forward starts with square(x), which throws on a
    # non-contiguous input (unary.cpp:19-21); the fused op keeps that error.
    x, w, _, _ = data(8, 12, F32, 302)
    base = np.ascontiguousarray(x.T)
    device = sp.Device.hip(0)
    view = sp.Tensor.from_numpy(base).to(device).transpose(0, 1)
    weight = sp.Tensor.from_numpy(w).to(device)
    with pytest.raises(ValueError, match="contiguous"):
        sp.rms_norm(view, weight)
    with pytest.raises(ValueError, match="contiguous"):
        R.rms_norm(R.RTensor.of(base).transpose(0, 1), R.RTensor.of(w))


# (RMSNorm on a transposed view is an error, tested above.)
# "narrowed" and "shifted" read the rows of a wider tensor in place (rows
# 536 elements apart, starting at element 4 or 1 of the row: vector and
# scalar paths).
LAYOUT_VIEW = {
    "contiguous": lambda t: t,
    "transposed": lambda t: t.transpose(0, 1),
    "narrowed": lambda t: t.narrow(1, 4, 520),
    "shifted": lambda t: t.narrow(1, 1, 520),
}


@pytest.mark.parametrize("center,layout", [(True, "contiguous"), (True, "transposed"),
                                           (False, "contiguous"), (True, "narrowed"),
                                           (True, "shifted")])
def test_norm_api_forward_backward(sp, center, layout):
    rows, n = 96, 520
    x, w, b, g = data(rows, n, F32, 300)
    if layout == "transposed":
        base = np.ascontiguousarray(x.T)
    elif layout in ("narrowed", "shifted"):
        start = 4 if layout == "narrowed" else 1
        base = np.random.default_rng(303).standard_normal((rows, n + 16)).astype(F32)
        base[:, start:start + n] = x
    else:
        base = x

    def build(lib, t):
        xv = LAYOUT_VIEW[layout](t[0])
        y = lib.layer_norm(xv, t[1], t[2], EPSILON) if center else lib.rms_norm(xv, t[1], EPSILON)
        loss = lib.sum(lib.multiply(y, t[3]))
        loss.backward()
        return y

    got_y, want_y, td, tr = api_both(sp, [base, w, b, g], build)
    assert_rows(got_y, want_y, n, F32, f"api y {layout}")
    cpu = sp.Device.cpu()
    dx_got, dx_want = td[0].grad().to(cpu).numpy(), tr[0].grad().numpy()
    if layout == "transposed":
        dx_got, dx_want = dx_got.T, dx_want.T
    elif layout in ("narrowed", "shifted"):
        start = 4 if layout == "narrowed" else 1
        outside = np.ones(n + 16, bool)
        outside[start:start + n] = False
        assert not dx_got[:, outside].any() and not dx_want[:, outside].any()
        dx_got, dx_want = dx_got[:, start:start + n], dx_want[:, start:start + n]
    # both gradients are back in [rows, n] orientation here
    assert_rows(dx_got, dx_want, n, F32, f"api dx {layout}", 16.0, dx_terms(g, w, x, center))
    for i in (1, 2) if center else (1,):
        got, want = td[i].grad().to(cpu).numpy(), tr[i].grad().numpy()
        scale = np.max(np.abs(want))
        assert np.max(np.abs(got - want)) <= 1e-6 * np.sqrt(rows * n) * 8 * scale, f"api grad {i}"
    if not center:  # the unused bias never received a gradient
        with pytest.raises(sp.LogicError):
            td[2].grad()


def test_norm_api_long_rows_use_composed_ops(sp):
    # rows longer than the fused kernels accept take the composed ops
    rows, n = 3, 20000
    x, w, b, g = data(rows, n, F32, 301)

    def build(lib, t):
        y = lib.rms_norm(t[0], t[1], EPSILON)
        lib.sum(lib.multiply(y, t[2])).backward()
        return y

    got_y, want_y, td, tr = api_both(sp, [x, w, g], build)
    assert_rows(got_y, want_y, n, F32, "composed y")
    assert_rows(td[0].grad().to(sp.Device.cpu()).numpy(), tr[0].grad().numpy(), n, F32,
                "composed dx", 16.0, dx_terms(g, w, x, False))


def test_norm_api_errors(sp):
    device = sp.Device.hip(0)
    x = sp.Tensor.from_numpy(np.ones((4, 8), F32)).to(device)
    w = sp.Tensor.from_numpy(np.ones(8, F32)).to(device)
    w_bad = sp.Tensor.from_numpy(np.ones(7, F32)).to(device)
    with pytest.raises(ValueError):
        sp.rms_norm(x, w_bad)
    with pytest.raises(ValueError):
        sp.layer_norm(x, w, w_bad)
    with pytest.raises(ValueError):
        sp.rms_norm(x, w, 0.0)
    with pytest.raises(ValueError):
        sp.rms_norm(x, sp.Tensor.from_numpy(np.ones(8, F64)).to(device))
    with pytest.raises(RuntimeError):
        sp.rms_norm(sp.Tensor.from_numpy(np.ones((4, 8), F32)), w)


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("center", [True, False])
@pytest.mark.parametrize("rows,n,pitch,first", [(64, 1024, 1040, 4), (33, 4096, 4100, 0),
                                                 (9, 1000, 1003, 3), (5, 8192, 8200, 8)])
def test_norm_row_stride_matches_contiguous(hip, dtype, center, rows, n, pitch, first):
    """Rows of a wider tensor (a sliced view's rows, `pitch` apart, starting
    `first` elements in).  Where every row start stays 16-byte aligned the
    kernels take the same vector path as for the rows made contiguous and
    must give the same bits, forward and backward; otherwise they take the
    scalar path, whose sums run in another order, and are held to the row
    tolerance against the contiguous results."""
    x, w, b, g = data(rows, n, dtype, 400 + n)
    wide = np.zeros((rows + 1) * pitch, dtype)
    for r in range(rows):
        wide[first + r * pitch:first + r * pitch + n] = x[r]
    y_ref, mu_ref, d_ref, (x_dev, mu, d) = forward_device(hip, x, w, b, center, dtype)
    wide_dev = dev(hip, wide)
    item = np.dtype(dtype).itemsize
    y, mu2, d2 = out_buf(hip, rows * n, dtype), out_buf(hip, rows, dtype), out_buf(hip, rows, dtype)
    hip.call("spar_hip_launch_norm_forward", y.ptr, mu2.ptr if center else None, d2.ptr,
             wide_dev.address(first * item), pitch, 1, dev(hip, w).ptr,
             dev(hip, b).ptr if center else None, rows, n, EPSILON, int(center), tag(dtype), 0)
    item_aligned = (first * item) % 16 == 0 and (pitch * item) % 16 == 0

    def same(got, want, what):
        if item_aligned:
            assert_bitexact(got, want, what)
        elif got.ndim == 2:
            assert_rows(got, want, n, dtype, what)
        else:
            bound = 1e-6 * np.sqrt(rows * n) * 8 * np.max(np.abs(want))
            assert np.max(np.abs(got - want)) <= bound, what

    same(y.to_numpy(dtype, (rows, n)), y_ref, "strided forward")
    same(d2.to_numpy(dtype, (rows,)), d_ref, "strided denominator")
    if center:
        same(mu2.to_numpy(dtype, (rows,)), mu_ref, "strided mean")
    outs = []
    for source, stride in ((x_dev.ptr, n), (wide_dev.address(first * item), pitch)):
        dx, dw, db = out_buf(hip, rows * n, dtype), out_buf(hip, n, dtype), out_buf(hip, n, dtype)
        hip.call("spar_hip_launch_norm_backward", dx.ptr, n, dw.ptr, db.ptr if center else None,
                 dev(hip, g).ptr, source, stride, 1, dev(hip, w).ptr, mu.ptr if center else None,
                 d.ptr, rows, n, int(center), tag(dtype), 0)
        outs.append([dx.to_numpy(dtype, (rows, n)), dw.to_numpy(dtype, (n,))] +
                    ([db.to_numpy(dtype, (n,))] if center else []))
    for a, c in zip(*outs):
        if item_aligned or a.ndim == 1:
            same(c, a, "strided backward")
        else:
            assert_rows(c, a, n, dtype, "strided backward dx", 16.0, dx_terms(g, w, x, center))


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("center", [True, False])
@pytest.mark.parametrize("rows,n,pitch,first", [
    (512, 1024, 512, 0),     # a transposed contiguous matrix: vector path, 2 splits
    (200, 520, 264, 4),      # a transposed block of a wider matrix
    (37, 300, 41, 3),        # unaligned: scalar loads and stores
    (8, 8192, 8, 0),         # few rows, long rows: 4 splits
    (130, 12, 130, 0),       # partial tiles in both directions, one split
    (3, 5, 7, 1),            # tiny and ragged
])
def test_norm_column_layout(hip, dtype, center, rows, n, pitch, first):
    """Rows that run down storage columns (x[p][q] = in[p + q * pitch]) against
    the row kernel on the same rows made contiguous.  The column path sums its
    statistics around a shift in double, the row kernel in T, so the two agree
    within the statistics' rounding: y within the row tolerance, mean and d
    within a few ulp of the row's scale."""
    check_column_layout(hip, dtype, center, rows, n, pitch, first)


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("center", [True, False])
def test_random_norm_column_layout(hip, dtype, center):
    """The column-layout forward over 20 random (rows, n, pitch, offset)
    layouts: partial tiles, pitches that are and are not multiples of the
    vector width, every split count the launcher picks."""
    rng = np.random.default_rng(96 + int(center) + (2 if dtype == F64 else 0))
    for case in range(20):
        while True:
            rows = int(rng.integers(1, 700))
            n = int(rng.integers(1, 3000))
            if rows * n <= (1 << 20):
                break
        pitch = rows + int(rng.integers(0, 40))
        first = int(rng.integers(0, 8))
        check_column_layout(hip, dtype, center, rows, n, pitch, first,
                            f"case {case}: rows {rows} n {n} pitch {pitch} first {first}")


def check_column_layout(hip, dtype, center, rows, n, pitch, first, what="column layout"):
    x, w, b, g = data(rows, n, dtype, 500 + rows + n)
    store = np.zeros(first + n * pitch, dtype)
    store[first:].reshape(n, pitch)[:, :rows] = x.T
    # highest element read: first + (rows - 1) + (n - 1) * pitch < store.size
    assert first + rows - 1 + (n - 1) * pitch < store.size
    y_ref, mu_ref, d_ref, _ = forward_device(hip, x, w, b, center, dtype)
    store_dev = dev(hip, store)
    item = np.dtype(dtype).itemsize
    y, mu, d = out_buf(hip, rows * n, dtype), out_buf(hip, rows, dtype), out_buf(hip, rows, dtype)
    hip.call("spar_hip_launch_norm_forward", y.ptr, mu.ptr if center else None, d.ptr,
             store_dev.address(first * item), 1, pitch, dev(hip, w).ptr,
             dev(hip, b).ptr if center else None, rows, n, EPSILON, int(center), tag(dtype), 0)
    assert_rows(y.to_numpy(dtype, (rows, n)), y_ref, n, dtype, what + " y")
    eps = np.finfo(dtype).eps
    scale = np.max(np.abs(x.astype(np.float64)), axis=1)
    got_d = d.to_numpy(dtype, (rows,)).astype(np.float64)
    assert np.all(np.abs(got_d - d_ref) <= 8 * eps * np.sqrt(n) * d_ref), what + " d"
    if center:
        got_mu = mu.to_numpy(dtype, (rows,)).astype(np.float64)
        assert np.all(np.abs(got_mu - mu_ref) <= 8 * eps * np.sqrt(n) * scale), what + " mean"
    # and against float64 statistics computed here
    x64 = x.astype(np.float64)
    mean64 = x64.mean(axis=1) if center else np.zeros(rows)
    d64 = np.sqrt(((x64 - mean64[:, None]) ** 2).mean(axis=1) + EPSILON)
    # float32: the double sums are exact to well below an ulp of T; float64:
    # they carry their own rounding, a random walk over the row
    allowance = 4.0 if dtype == F32 else 8.0 * np.sqrt(n)
    assert np.all(np.abs(got_d - d64) <= allowance * eps * d64), what + " d vs float64"


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("center", [True, False])
@pytest.mark.parametrize("layout,rows,n,stride,first", [
    ("rows", 64, 2048, 2304, 256),   # a block of a wider gradient, 16-byte aligned
    ("rows", 37, 300, 309, 5),       # unaligned rows: scalar stores
    ("columns", 256, 512, 320, 64),  # q columns further apart than rows
    ("columns", 37, 300, 41, 3),     # unaligned
])
def test_norm_backward_strided_input_gradient(hip, dtype, center, layout, rows, n, stride,
                                              first):
    """dx written into a wider buffer: rows `stride` apart (row layout) or
    element (p, q) at first + p + q * stride (column layout).  The block holds
    exactly the values of the packed write (same kernels, same order), and
    every element around it keeps the sentinel it was filled with."""
    x, w, b, g = data(rows, n, dtype, 900 + rows + n)
    _, _, _, (x_dev, mu, d) = forward_device(hip, x, w, b, center, dtype)
    item = np.dtype(dtype).itemsize
    if layout == "rows":
        source, row_stride, column_stride, packed_stride = x_dev.ptr, n, 1, n
        size = first + (rows - 1) * stride + n
    else:
        store = np.zeros(n * rows, dtype)
        store.reshape(n, rows)[:, :] = x.T
        source, row_stride, column_stride, packed_stride = dev(hip, store).ptr, 1, rows, rows
        size = first + rows + (n - 1) * stride
    g_dev, w_dev = dev(hip, g), dev(hip, w)
    sentinel = np.full(size, -7.25, dtype)
    wide = dev(hip, sentinel)
    # the packed write starts at the same offset, so both take the same
    # (vector or scalar) kernel and sum in the same order
    packed = out_buf(hip, first + rows * n, dtype)
    dws = []
    for dx_ptr, dx_stride in ((packed.address(first * item), packed_stride),
                              (wide.address(first * item), stride)):
        dw, db = out_buf(hip, n, dtype), out_buf(hip, n, dtype)
        hip.call("spar_hip_launch_norm_backward", dx_ptr, dx_stride,
                 dw.ptr, db.ptr if center else None, g_dev.ptr, source, row_stride,
                 column_stride, w_dev.ptr, mu.ptr if center else None, d.ptr, rows, n,
                 int(center), tag(dtype), 0)
        dws.append(dw.to_numpy(dtype, (n,)))
    flat = packed.to_numpy(dtype, (first + rows * n,))[first:]
    got = wide.to_numpy(dtype, (size,))
    written = np.zeros(size, bool)
    p_idx, q_idx = np.meshgrid(np.arange(rows), np.arange(n), indexing="ij")
    if layout == "rows":
        where = first + p_idx * stride + q_idx
        want = flat.reshape(rows, n)
    else:
        where = first + p_idx + q_idx * stride
        want = flat.reshape(n, rows).T
    written[where.ravel()] = True
    assert_bitexact(got[where], want, f"strided dx {layout}")
    assert np.all(got[~written] == dtype(-7.25)), "elements around the block were written"
    assert_bitexact(dws[1], dws[0], "d weight")


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("center", [True, False])
@pytest.mark.parametrize("rows,n,pitch,first", [
    (512, 1024, 512, 0),     # a transposed contiguous matrix: whole tiles
    (200, 520, 264, 4),      # a transposed block of a wider matrix: partial tiles
    (37, 300, 41, 3),        # unaligned: scalar loads and stores
    (8, 8192, 8, 0),         # few rows, long rows: one p tile, many q splits
    (1000, 12, 1000, 0),     # many rows, short rows: one q tile
    (3, 5, 7, 1),            # tiny and ragged
    # long columns ending in a partial p tile, x within the sums pass's cache
    # budget (float32 4800) or over it (the others)
    (4800, 8192, 4800, 0),
    (5280, 8192, 5280, 0),
])
def test_norm_backward_column_layout(hip, dtype, center, rows, n, pitch, first):
    """The backward over rows that run down storage columns writes dx packed
    in that layout (dx[p + q * rows]).  Against the row kernel on the same
    rows made contiguous, with the same saved statistics: the two sum in
    different orders, so dx within the dx row tolerance and the parameter
    gradients within red(rows) of their terms."""
    x, w, b, g = data(rows, n, dtype, 700 + rows + n)
    store = np.zeros(first + n * pitch, dtype)
    store[first:].reshape(n, pitch)[:, :rows] = x.T
    assert first + rows - 1 + (n - 1) * pitch < store.size
    _, _, _, (x_dev, mu, d) = forward_device(hip, x, w, b, center, dtype)
    store_dev = dev(hip, store)
    item = np.dtype(dtype).itemsize
    g_dev, w_dev = dev(hip, g), dev(hip, w)
    outs = []
    for source, row_stride, column_stride in ((x_dev.ptr, n, 1),
                                              (store_dev.address(first * item), 1, pitch)):
        dx, dw, db = out_buf(hip, rows * n, dtype), out_buf(hip, n, dtype), out_buf(hip, n, dtype)
        hip.call("spar_hip_launch_norm_backward", dx.ptr, n if column_stride == 1 else rows,
                 dw.ptr, db.ptr if center else None,
                 g_dev.ptr, source, row_stride, column_stride, w_dev.ptr,
                 mu.ptr if center else None, d.ptr, rows, n, int(center), tag(dtype), 0)
        got = dx.to_numpy(dtype, (rows * n,))
        got = got.reshape(rows, n) if column_stride == 1 else got.reshape(n, rows).T
        outs.append((got, dw.to_numpy(dtype, (n,)), db.to_numpy(dtype, (n,)) if center else None))
    (dx_rows, dw_rows, db_rows), (dx_cols, dw_cols, db_cols) = outs
    what = f"column backward {rows}x{n} {np.dtype(dtype).name} center={center}"
    assert_rows(dx_cols, dx_rows, n, dtype, what + " dx", 16.0, dx_terms(g, w, x, center))
    x64 = x.astype(np.float64)
    xc = x64 - (x64.mean(axis=1, keepdims=True) if center else 0)
    xhat = xc / np.sqrt(np.mean(xc * xc, axis=1, keepdims=True) + EPSILON)
    terms = np.abs(g.astype(np.float64) * xhat)
    bound = 8e-6 * np.sqrt(max(rows, n)) * np.sum(terms, axis=0) + 1e-30
    assert np.all(np.abs(dw_cols.astype(np.float64) - dw_rows) <= bound), what + " d weight"
    if center:
        bound = 8e-6 * np.sqrt(rows) * np.sum(np.abs(g.astype(np.float64)), axis=0) + 1e-30
        assert np.all(np.abs(db_cols.astype(np.float64) - db_rows) <= bound), what + " d bias"


def test_layer_norm_transposed_gradient_is_packed(sp):
    """The gradient of a transposed view's LayerNorm reaches the base as a
    contiguous [n, rows] tensor: the norm's backward writes it packed in the
    column layout, and transpose's backward passes it on without a copy."""
    rows, n = 96, 160
    rng = np.random.default_rng(5)
    base = rng.standard_normal((n, rows)).astype(F32)
    w = rng.uniform(0.5, 1.5, n).astype(F32)
    bias = rng.uniform(-0.1, 0.1, n).astype(F32)
    g = rng.standard_normal((rows, n)).astype(F32)

    def build(lib, t):
        y = lib.layer_norm(t[0].transpose(0, 1), t[1], t[2], EPSILON)
        lib.sum(lib.multiply(y, t[3])).backward()
        return y

    got_y, want_y, td, tr = api_both(sp, [base, w, bias, g], build)
    assert_rows(got_y, want_y, n, F32, "transposed y")
    cpu = sp.Device.cpu()
    grad = td[0].grad()
    assert grad.is_contiguous() and tuple(grad.shape) == (n, rows)
    assert_rows(grad.to(cpu).numpy().T, tr[0].grad().numpy().T, n, F32, "transposed dx", 16.0,
                dx_terms(g, w, base.T, True))


@pytest.mark.parametrize("shape", [(12, 8, 300), (5, 7, 64)])
def test_layer_norm_api_batched_column_layout(sp, shape):
    """A rank-3 view whose rows run down storage columns: base [n, A, B]
    permuted to [A, B, n] has leading axes contiguous among themselves and
    the last axis A*B apart, so the fused forward reads it in the column
    layout.  Forward and backward against the oracle's composition."""
    a, b, n = shape
    rng = np.random.default_rng(sum(shape))
    base = rng.standard_normal((n, a, b)).astype(F32)
    w = rng.uniform(0.5, 1.5, n).astype(F32)
    bias = rng.uniform(-0.1, 0.1, n).astype(F32)
    g = rng.standard_normal((a, b, n)).astype(F32)

    def build(lib, t):
        y = lib.layer_norm(t[0].permute([1, 2, 0]), t[1], t[2], EPSILON)
        lib.sum(lib.multiply(y, t[3])).backward()
        return y

    got_y, want_y, td, tr = api_both(sp, [base, w, bias, g], build)
    rows_got, rows_want = got_y.reshape(-1, n), want_y.reshape(-1, n)
    assert_rows(rows_got, rows_want, n, F32, "batched column y")
    cpu = sp.Device.cpu()
    dx_got = td[0].grad().to(cpu).numpy().transpose(1, 2, 0).reshape(-1, n)
    dx_want = tr[0].grad().numpy().transpose(1, 2, 0).reshape(-1, n)
    x_rows = base.transpose(1, 2, 0).reshape(-1, n)
    assert_rows(dx_got, dx_want, n, F32, "batched column dx", 16.0,
                dx_terms(g.reshape(-1, n), w, x_rows, True))
    for i in (1, 2):
        got, want = td[i].grad().to(cpu).numpy(), tr[i].grad().numpy()
        scale = np.max(np.abs(want))
        assert np.max(np.abs(got - want)) <= 1e-6 * np.sqrt(a * b * n) * 8 * scale, f"grad {i}"
