"""The fused norms' backward with the output gradient given as factor x value.

loss = sum(y * c) with c needing no gradient hands y the gradient value * c,
value the single element of sum's broadcast gradient.  The engine passes the
norm's backward (c, value) instead of materialising the product
(spar_hip_launch_norm_backward_scaled), and the kernels form value * c[i]
themselves.  The bar is bit-identity with the unscaled backward fed the
materialised product:

  * kernel level: spar_hip_launch_norm_backward_scaled(c, value) against
    spar_hip_launch_norm_backward(value * c), the product formed on the host
    by numpy (one IEEE multiply, value on the left as the multiply op has
    it), in both layouts and in the vector and scalar paths;
  * API level: the same forward and loss with c not requiring a gradient
    (the scaled hand-over, counted by autograd_counters) and with c requiring
    one (the product op's own rule runs, since the product then has two
    tracked inputs): the gradients of x, weight and bias agree bit for bit.
"""
import numpy as np
import pytest

from tests.helpers import assert_bitexact

pytestmark = pytest.mark.gpu

F32, F64 = np.float32, np.float64
EPSILON = 1.0e-5

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


def tag(dtype):
    return 0 if np.dtype(dtype) == F32 else 1


SCALED_CASES = [
    ("rows", 64, 2048),      # vector rows, pipelined kernel (float32)
    ("rows", 37, 301),       # extent not a multiple of 4: scalar path
    ("rows", 9, 12000),      # long rows: the plain kernel (float32 only: float64 rows
                             # take at most 8192 elements)
    ("columns", 256, 512),   # transposed matrix: whole tiles
    ("columns", 200, 520),   # partial tiles
    ("columns", 37, 300),    # unaligned: scalar tiles
]


@pytest.mark.parametrize("dtype,layout,rows,n", [
    (dtype, *case) for dtype in (F32, F64) for case in SCALED_CASES
    if not (dtype == F64 and case[2] > 8192)])
@pytest.mark.parametrize("center", [True, False])
@pytest.mark.parametrize("value", [1.0, 3.0, -0.375, np.inf])
def test_scaled_backward_matches_materialised_product(hip, dtype, center, layout, rows, n,
                                                      value):
    rng = np.random.default_rng(rows * 7 + n)
    x = (rng.standard_normal((rows, n)) * 2 + 0.5).astype(dtype)
    w = rng.uniform(0.5, 1.5, n).astype(dtype)
    b = rng.uniform(-0.1, 0.1, n).astype(dtype)
    c = rng.standard_normal((rows, n)).astype(dtype)
    c[0, :3] = 0.0  # inf * 0 is NaN: absent elements must stay zero, present ones NaN
    c[-1, -1] = -0.0
    scale = np.array([value], dtype)
    with np.errstate(invalid="ignore"):  # inf * 0 is the intended NaN
        product = scale[0] * c  # one IEEE multiply per element, value on the left
    assert product.dtype == np.dtype(dtype)
    # forward statistics
    y, mu, d = out_buf(hip, rows * n, dtype), out_buf(hip, rows, dtype), out_buf(hip, rows, dtype)
    if layout == "rows":
        source = dev(hip, x)
        row_stride, column_stride, dx_stride = n, 1, n
    else:
        source = dev(hip, np.ascontiguousarray(x.T))  # x[p][q] at p + q * rows
        row_stride, column_stride, dx_stride = 1, rows, rows
    w_dev, b_dev = dev(hip, w), dev(hip, b)
    hip.call("spar_hip_launch_norm_forward", y.ptr, mu.ptr if center else None, d.ptr,
             source.ptr, row_stride, column_stride, w_dev.ptr, b_dev.ptr if center else None,
             rows, n, EPSILON, int(center), tag(dtype), 0)
    outs = []
    for scaled in (False, True):
        dx, dw, db = (out_buf(hip, rows * n, dtype), out_buf(hip, n, dtype),
                      out_buf(hip, n, dtype))
        common = (source.ptr, row_stride, column_stride, w_dev.ptr, mu.ptr if center else None,
                  d.ptr, rows, n, int(center), tag(dtype), 0)
        if scaled:
            hip.call("spar_hip_launch_norm_backward_scaled", dx.ptr, dx_stride, dw.ptr,
                     db.ptr if center else None, dev(hip, c).ptr, dev(hip, scale).ptr, *common)
        else:
            hip.call("spar_hip_launch_norm_backward", dx.ptr, dx_stride, dw.ptr,
                     db.ptr if center else None, dev(hip, product).ptr, *common)
        outs.append((dx.to_numpy(dtype, (rows * n,)), dw.to_numpy(dtype, (n,)),
                     db.to_numpy(dtype, (n,)) if center else None))
    what = f"{layout} {rows}x{n} {np.dtype(dtype).name} center={center} value={value}"
    assert_bitexact(outs[1][0], outs[0][0], what + " dx")
    assert_bitexact(outs[1][1], outs[0][1], what + " d weight")
    if center:
        assert_bitexact(outs[1][2], outs[0][2], what + " d bias")


def test_scaled_backward_requires_a_scale(hip):
    buf = out_buf(hip, 64, F32)
    status = hip.status_of("spar_hip_launch_norm_backward_scaled", buf.ptr, 8, buf.ptr,
                             buf.ptr, buf.ptr, None, buf.ptr, 8, 1, buf.ptr, buf.ptr, buf.ptr,
                             4, 8, 1, 0, 0)
    assert status.code == 1


# ------------------------------------------------------------------ API

@pytest.fixture(scope="module")
def sp():
    from spar_amd import spar

    if spar.hip_device_count() < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    return spar


VIEWS = {
    "contiguous": (lambda rows, n: (rows, n), lambda t, rows, n: t),
    "transposed": (lambda rows, n: (n, rows), lambda t, rows, n: t.transpose(0, 1)),
    "sliced": (lambda rows, n: (rows + 24, n + 40),
               lambda t, rows, n: t.narrow(0, 16, rows).narrow(1, 8, n)),
}


# rms_norm takes contiguous inputs only
@pytest.mark.parametrize("center,view", [(True, "contiguous"), (True, "transposed"),
                                         (True, "sliced"), (False, "contiguous")])
@pytest.mark.parametrize("loss_scale", [None, 2.5])
def test_api_scaled_hand_over_is_bit_identical(sp, center, view, loss_scale):
    """loss = sum(y * c) (times loss_scale): with c a constant the product's
    gradient reaches the norm as (c, value); with c tracked the product's own
    rule materialises it.  Same gradients, bit for bit."""
    rows, n = 96, 520
    shape_of, view_of = VIEWS[view]
    rng = np.random.default_rng(41 + rows + (loss_scale is not None))
    base = rng.standard_normal(shape_of(rows, n)).astype(F32)
    w = rng.uniform(0.5, 1.5, n).astype(F32)
    b = rng.uniform(-0.1, 0.1, n).astype(F32)
    c = rng.standard_normal((rows, n)).astype(F32)
    device, cpu = sp.Device.hip(0), sp.Device.cpu()

    def run(c_tracked):
        leaves = [sp.Tensor.from_numpy(a).to(device) for a in (base, w, b)]
        for leaf in leaves:
            leaf.set_requires_grad(True)
        constant = sp.Tensor.from_numpy(c).to(device)
        if c_tracked:
            constant.set_requires_grad(True)
        x = view_of(leaves[0], rows, n)
        y = sp.layer_norm(x, leaves[1], leaves[2], EPSILON) if center else \
            sp.rms_norm(x, leaves[1], EPSILON)
        loss = sp.sum(sp.multiply(y, constant))
        if loss_scale is not None:
            loss = sp.multiply_scalar(loss, loss_scale)
        before = sp.autograd_counters()["scaled_gradients"]
        loss.backward()
        handed = sp.autograd_counters()["scaled_gradients"] - before
        grads = [leaf.grad().to(cpu).numpy() for leaf in (leaves if center else leaves[:2])]
        return grads, handed

    scaled, handed = run(False)
    plain, plain_handed = run(True)
    assert handed == 1 and plain_handed == 0
    for k, (got, want) in enumerate(zip(scaled, plain)):
        assert_bitexact(got, want, f"{view} center={center} scale={loss_scale} grad {k}")
