"""Kernel-level parity: every C-ABI launcher against the oracle.

Inputs are seeded and identical on both sides (host bytes copied to the
device).  Tolerance classes are defined in tests/helpers.py.
"""
import ctypes

import numpy as np
import pytest

from oracle import ops as ref
from tests.helpers import (assert_bitexact, assert_red, assert_ulp, special_values)

pytestmark = pytest.mark.gpu

F32, F64 = np.float32, np.float64
DTYPES = [F32, F64]


def tag(dtype):
    return 0 if np.dtype(dtype) == np.float32 else 1


# Device buffers stay alive until the test ends: a buffer freed early would
# return its block to the caching allocator and the next upload could reuse it.
_alive = []


@pytest.fixture(autouse=True)
def _release_buffers():
    yield
    _alive.clear()


def dev(hip, array):
    buffer = hip.DeviceBuffer.from_numpy(np.ascontiguousarray(array))
    _alive.append(buffer)
    return buffer


def out_buf(hip, shape, dtype):
    n = int(np.prod(shape, dtype=np.int64))
    buffer = hip.DeviceBuffer(max(n, 1) * np.dtype(dtype).itemsize)
    _alive.append(buffer)
    return buffer


def inputs(seed, n, dtype, with_specials=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(dtype)
    if with_specials and n >= 64:
        sp = special_values(dtype)
        x[: sp.size] = sp
        rng.shuffle(x)
    return x


# ------------------------------------------------------------ elementwise

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 3, 4, 7, 1000, 4096, 65537, 1 << 20])
@pytest.mark.parametrize("op", list(ref.BINARY))
def test_binary_contiguous_bitexact(hip, dtype, n, op):
    a = inputs(1, n, dtype)
    b = inputs(2, n, dtype)
    out = out_buf(hip, (n,), dtype)
    hip.call("spar_hip_launch_binary", out.ptr, dev(hip, a).ptr, dev(hip, b).ptr, n, tag(dtype),
             hip.BINARY_OPS[op], 0)
    assert_bitexact(out.to_numpy(dtype, (n,)), ref.binary(a, b, op), f"{op} n={n}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("op", ["add", "subtract", "multiply", "divide"])
@pytest.mark.parametrize("value", [0.1, -3.0, 1e-3, 2.5e38, 0.0])
def test_scalar_bitexact(hip, dtype, op, value):
    n = 10007
    a = inputs(3, n, dtype)
    out = out_buf(hip, (n,), dtype)
    hip.call("spar_hip_launch_scalar", out.ptr, dev(hip, a).ptr, n, tag(dtype),
             hip.BINARY_OPS[op], value, 0)
    assert_bitexact(out.to_numpy(dtype, (n,)), ref.scalar(a, op, value), f"{op} {value}")


EXACT_UNARY = ["negate", "square", "reciprocal", "sqrt"]
TRANSCENDENTAL = ["exp", "log", "sigmoid", "silu", "tanh", "gelu"]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("op", EXACT_UNARY + TRANSCENDENTAL)
def test_unary(hip, dtype, op):
    n = 200003
    with np.errstate(over="ignore"):
        a = inputs(4, n, dtype) * dtype(4)
    if op in ("log", "sqrt"):
        a = np.abs(a)
        a[:5] = [0.0, -0.0, -1.0, np.inf, np.nan]
    out = out_buf(hip, (n,), dtype)
    hip.call("spar_hip_launch_unary", out.ptr, dev(hip, a).ptr, n, tag(dtype), hip.UNARY_OPS[op], 0)
    got = out.to_numpy(dtype, (n,))
    want = ref.unary(a, op)
    if op in EXACT_UNARY:
        assert_bitexact(got, want, op)
    else:
        # float32: <= 2 ulp.  float64 composites (sigmoid/silu/gelu) chain two
        # libm results with no wider type to evaluate in: <= 4 ulp.
        composite = op in ("sigmoid", "silu", "gelu")
        assert_ulp(got, want, 4 if (dtype == F64 and composite) else 2, op)


def test_gelu_float32_sweep(hip):
    """Every 256th float32 bit pattern (2^24 inputs spanning every exponent
    and both signs, with the infinities and NaNs) through GELU and its
    derivative against the oracle's double-precision definition.  GELU is
    within 1 ulp everywhere; the derivative is within 1 ulp except for x in
    [-0.7576, -0.7473], where Phi(x) + x phi(x) cancels near its root and the
    bound is 2.4e-10 absolute (both measured on all 2^32 inputs on the CPU)."""
    bits = (np.arange(1 << 24, dtype=np.uint64) * 256 + 77).astype(np.uint32)
    x = bits.view(F32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -15.0, 15.0,
                                     -0.7518, np.finfo(F32).tiny, -np.finfo(F32).max], F32)])
    n = x.size
    out = out_buf(hip, (n,), F32)
    d = dev(hip, x)
    hip.call("spar_hip_launch_unary", out.ptr, d.ptr, n, 0, hip.GELU, 0)
    assert_ulp(out.to_numpy(F32, (n,)), ref.unary(x, "gelu"), 1, "gelu sweep")
    hip.call("spar_hip_launch_unary", out.ptr, d.ptr, n, 0, hip.GELU_DERIVATIVE, 0)
    got = out.to_numpy(F32, (n,))
    want = ref.unary(x, "gelu_derivative")
    assert np.array_equal(np.isnan(got), np.isnan(want)), "gelu' NaN positions"
    finite = np.isfinite(want)
    assert np.array_equal(got[~finite & ~np.isnan(want)], want[~finite & ~np.isnan(want)])
    err = np.abs(got[finite].astype(np.float64) - want[finite].astype(np.float64))
    ulp = np.spacing(np.abs(want[finite])).astype(np.float64)
    near_root = (x[finite] >= -0.7576) & (x[finite] <= -0.7473)
    bad = (err > ulp) & ~(near_root & (err <= 2.4e-10))
    assert not bad.any(), f"gelu' sweep: {int(bad.sum())} outside the bound, e.g. x={x[finite][bad][:3]}"


def test_gelu_large_sweep(hip):
    """Every 128th float32 bit pattern (2^25 inputs, every exponent and both
    signs) plus a ragged tail of 7 elements through the contiguous GELU kernel
    (32 tiles per workgroup, then the leftover vectors and elements): within 1
    ulp of the double definition, and the same bits as a call on the first
    2^24 + 3 of them, whose tiles and leftovers fall elsewhere."""
    bits = (np.arange(1 << 25, dtype=np.uint64) * 128 + 45).astype(np.uint32)
    x = np.concatenate([bits.view(F32), np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -15.0,
                                                  15.0], F32)])
    n = x.size
    assert n >= 1 << 25 and n % 4 == 3
    d = dev(hip, x)
    out = out_buf(hip, (n,), F32)
    hip.call("spar_hip_launch_unary", out.ptr, d.ptr, n, 0, hip.GELU, 0)
    full = out.to_numpy(F32, (n,))
    assert_ulp(full, ref.unary(x, "gelu"), 1, "gelu large sweep")
    m = (1 << 24) + 3
    small = out_buf(hip, (m,), F32)
    hip.call("spar_hip_launch_unary", small.ptr, d.ptr, m, 0, hip.GELU, 0)
    assert_bitexact(small.to_numpy(F32, (m,)), full[:m], "gelu shorter call")


def test_exp_clipped_config_range(hip):
    # exp over N(0,1) clipped to [-10, 10], the elementwise benchmark input
    x = np.clip(np.random.default_rng(5).standard_normal(1 << 20), -10, 10).astype(F32)
    out = out_buf(hip, x.shape, F32)
    hip.call("spar_hip_launch_unary", out.ptr, dev(hip, x).ptr, x.size, 0, hip.EXP, 0)
    assert_ulp(out.to_numpy(F32, x.shape), ref.unary(x, "exp"), 2, "exp")


def test_unaligned_pointers_take_scalar_path(hip):
    n = 4099
    a = inputs(6, n + 1, F32)
    b = inputs(7, n + 1, F32)
    da, db = dev(hip, a), dev(hip, b)
    out = out_buf(hip, (n + 1,), F32)
    # offset every pointer by one element (4 bytes): not 16-byte aligned
    hip.call("spar_hip_launch_binary", out.address(4), da.address(4), db.address(4), n, 0,
             hip.ADD, 0)
    got = out.to_numpy(F32, (n + 1,))[1:]
    assert_bitexact(got, ref.binary(a[1:], b[1:], "add"), "unaligned add")


@pytest.mark.parametrize("n", [1, 3, 1027, 4099, 2 * 512 * 2 * 4 + 13, 1 << 20, 257 * 4096 + 3,
                               3 * 256 * 4096 + 23])
def test_gelu_layouts_agree(hip, n):
    """GELU float32 reads its tail table from LDS in the contiguous kernel
    (whole tiles, leftover vectors, leftover elements) and from global memory
    on the unaligned scalar path and on strided views: the same bits, within
    1 ulp of the double definition."""
    x = np.random.default_rng(n).standard_normal(n + 1).astype(F32) * 4
    x[: min(n, 8)] = np.array([0.0, -0.0, 15.0, -15.0, 15.5, -15.5, np.inf, -np.inf], F32)[: min(n, 8)]
    d = dev(hip, x)
    aligned, shifted = out_buf(hip, (n + 1,), F32), out_buf(hip, (n + 1,), F32)
    hip.call("spar_hip_launch_unary", aligned.ptr, d.ptr, n, 0, hip.GELU, 0)
    hip.call("spar_hip_launch_unary", shifted.address(4), d.address(4), n, 0, hip.GELU, 0)
    got = aligned.to_numpy(F32, (n + 1,))[:n]
    got_shifted = shifted.to_numpy(F32, (n + 1,))[1:]
    want = ref.unary(x, "gelu")
    assert_ulp(got, want[:n], 1, "gelu contiguous")
    assert_ulp(got_shifted, want[1:], 1, "gelu unaligned")
    # the element both calls computed from x[k] for 1 <= k < n: same bits
    assert_bitexact(got[1:], got_shifted[: n - 1], "gelu LDS table vs global table")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("outer,extent,inner,start,length", [
    (3, 10, 1, 2, 5),        # last axis, unaligned window: element path
    (4, 16, 1, 4, 8),        # last axis, aligned window: 16-byte groups (float32)
    (5, 7, 8, 2, 3),         # inner rows of 8
    (2, 9, 3, 0, 9),         # the whole axis
    (6, 5, 4, 5, 0),         # an empty window at the end: all zeros
    (64, 1000, 36, 100, 800),
    (512, 9216, 1, 512, 8192),
])
def test_window_embed(hip, dtype, outer, extent, inner, start, length):
    """narrow's gradient scattered into a zeroed tensor of the base's shape in
    one pass, against numpy (bit copies, so exact)."""
    rng = np.random.default_rng(outer + extent + inner)
    window = rng.standard_normal((outer, length, inner)).astype(dtype)
    want = np.zeros((outer, extent, inner), dtype)
    want[:, start:start + length, :] = window
    out = out_buf(hip, want.shape, dtype)
    hip.call("spar_hip_launch_fill", out.ptr, want.size, tag(dtype), 7.0, 0)  # not zero beforehand
    src = dev(hip, window) if window.size else None
    hip.call("spar_hip_launch_window_embed", out.ptr, src.ptr if src else None, outer, extent,
             inner, start, length, np.dtype(dtype).itemsize, 0)
    assert_bitexact(out.to_numpy(dtype, want.shape), want, "window embed")


def test_window_embed_rejects_bad_arguments(hip):
    lib = hip.load()
    p = out_buf(hip, (64,), F32).ptr
    for args in [(p, p, 2, 4, 1, 5, 0, 4, 0),     # start past the axis
                 (p, p, 2, 4, 1, 2, 3, 4, 0),     # window past the axis
                 (p, p, 2, 4, 1, 0, 4, 2, 0),     # element size 2
                 (p, p, 1 << 20, 1 << 12, 1, 0, 1, 4, 0)]:  # more than 2^31 - 1 elements
        assert lib.spar_hip_launch_window_embed(*args).code == 1, args


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("extents,box", [
    ((4608, 9216), ((256, 4096), (512, 8192))),      # a block of a matrix, 16-byte groups
    ((13, 17, 9), ((3, 5), (3, 10), (1, 6))),         # three boxed axes, element path
    ((6, 1, 8, 12), ((1, 4), (0, 1), (0, 8), (4, 8))),  # unit and whole axes coalesced
    ((5, 7), ((0, 5), (0, 7))),                       # the whole tensor
    ((2, 3, 4, 5, 6), ((1, 1), (0, 3), (0, 4), (0, 5), (2, 3))),  # three whole axes merged
])
def test_box_embed(hip, dtype, extents, box):
    """A box of several axes scattered into zeros in one pass (a chain of
    narrows' gradient), against numpy (bit copies, so exact)."""
    lengths = tuple(length for _, length in box)
    rng = np.random.default_rng(sum(extents))
    inner = rng.standard_normal(lengths).astype(dtype)
    want = np.zeros(extents, dtype)
    want[tuple(slice(start, start + length) for start, length in box)] = inner
    out = out_buf(hip, want.shape, dtype)
    hip.call("spar_hip_launch_fill", out.ptr, want.size, tag(dtype), 7.0, 0)  # not zero beforehand
    src = dev(hip, inner)
    arrays = [np.array(v, dtype=np.uint64) for v in (extents, [b[0] for b in box], lengths)]
    hip.call("spar_hip_launch_box_embed", out.ptr, src.ptr, len(extents),
             *[a.ctypes.data for a in arrays], np.dtype(dtype).itemsize, 0)
    assert_bitexact(out.to_numpy(dtype, want.shape), want, "box embed")
    # input null: only the zeros around the box; the box keeps what it held
    hip.call("spar_hip_launch_fill", out.ptr, want.size, tag(dtype), 7.0, 0)
    hip.call("spar_hip_launch_box_embed", out.ptr, None, len(extents),
             *[a.ctypes.data for a in arrays], np.dtype(dtype).itemsize, 0)
    border = np.zeros(extents, dtype)
    border[tuple(slice(start, start + length) for start, length in box)] = 7.0
    assert_bitexact(out.to_numpy(dtype, want.shape), border, "box border")


def test_box_embed_rejects_bad_arguments(hip):
    lib = hip.load()
    p = out_buf(hip, (4096,), F32).ptr

    def call(extents, starts, lengths, size=4):
        arrays = [np.array(v, dtype=np.uint64) for v in (extents, starts, lengths)]
        return lib.spar_hip_launch_box_embed(p, p, len(extents), *[a.ctypes.data for a in arrays],
                                             size, 0).code

    assert call((4, 8), (0, 6), (4, 3)) == 1                  # box past the axis
    assert call((4, 8), (0, 2), (4, 3), size=2) == 1          # element size 2
    assert call((4, 8), (0, 2), (0, 3)) == 1                  # empty box: caller fills zeros
    assert call((4, 4, 4, 4, 4), (1,) * 5, (2,) * 5) == 1     # five boxed axes
    assert call((1 << 16, 1 << 16), (0, 0), (1, 1)) == 1      # more than 2^31 - 1 elements
    assert call((4, 8), (1, 2), (2, 3)) == 0
    arrays = [np.array(v, dtype=np.uint64) for v in ((4, 8), (0, 2), (0, 3))]
    assert lib.spar_hip_launch_box_embed(p, None, 2, *[a.ctypes.data for a in arrays], 4,
                                         0).code == 1  # empty box, border only


@pytest.mark.parametrize("dtype", DTYPES)
def test_fill_add_in_place_zero(hip, dtype):
    n = 12345
    d = out_buf(hip, (n,), dtype)
    hip.call("spar_hip_launch_fill", d.ptr, n, tag(dtype), 1.0, 0)
    assert np.all(d.to_numpy(dtype, (n,)) == 1)
    src = inputs(8, n, dtype, with_specials=False)
    want = np.ones(n, dtype)
    ref.add_in_place(want, src)
    hip.call("spar_hip_launch_add_in_place", d.ptr, dev(hip, src).ptr, n, tag(dtype), 0)
    assert_bitexact(d.to_numpy(dtype, (n,)), want, "add_in_place")
    hip.call("spar_hip_zero", d.ptr, n * np.dtype(dtype).itemsize, 0)
    assert np.all(d.to_numpy(dtype, (n,)) == 0)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("scale", [1.0, 0.25, 1.0 / 3.0, 1.0 / 4096.0, -2.5])
def test_fill_from_scalar_multiplies_like_reference(hip, dtype, scale):
    # the reference kernel writes scalar[0] * (T)scale (cuda_kernels.cu:249-257)
    g = np.array([0.7], dtype)
    n = 1000
    out = out_buf(hip, (n,), dtype)
    hip.call("spar_hip_launch_fill_from_scalar", out.ptr, dev(hip, g).ptr, n, tag(dtype), scale, 0)
    want = np.full(n, g[0] * dtype(scale), dtype)
    assert_bitexact(out.to_numpy(dtype, (n,)), want, "fill_from_scalar")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("divisor", [1.0, 3.0, 1000.0, 4096.0, 67108864.0])
def test_fill_from_scalar_divided_like_cpu(hip, dtype, divisor):
    g = np.array([0.7], dtype)
    n = 1000
    out = out_buf(hip, (n,), dtype)
    hip.call("spar_hip_launch_fill_from_scalar_divided", out.ptr, dev(hip, g).ptr, n, tag(dtype),
             divisor, 0)
    # mean backward on the CPU: g / (T)n (ops/reduction.cpp:263-277)
    want = np.full(n, g[0] / dtype(divisor), dtype)
    assert_bitexact(out.to_numpy(dtype, (n,)), want, "fill_from_scalar_divided")
    if divisor == 1000.0 and dtype == np.float32:
        # the two forms round apart here: 0.7f / 1000 != 0.7f * (float)(1 / 1000)
        assert np.float32(0.7) * np.float32(1e-3) != want[0]


# --------------------------------------------------------------- layouts

def check_span(base, shape, strides, offset):
    """Host-side guard: every element of the view lies inside `base`."""
    assert offset >= 0, f"view starts before its base (offset {offset})"
    last = offset + sum((d - 1) * s for d, s in zip(shape, strides) if d > 0)
    assert all(s >= 0 for s in strides) and last < base.size, \
        f"view reaches element {last} of a {base.size}-element base"


def strided_copy(hip, base, view, dtype):
    """Runs spar_hip_launch_strided_copy on `view`, a numpy view of `base`."""
    item = base.itemsize
    offset = (view.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // item
    strides = [s // item for s in view.strides]
    check_span(base, view.shape, strides, offset)
    db = dev(hip, base)
    out = out_buf(hip, view.shape, dtype)
    hip.call("spar_hip_launch_strided_copy", out.ptr, db.ptr, view.ndim, hip.u64_array(view.shape),
             hip.u64_array(strides), offset, view.size, item, 0)
    return out.to_numpy(dtype, view.shape)


def views_of(base2d):
    yield "transpose", base2d.T
    yield "slice", base2d[3:, 5:-2]
    yield "slice_step", base2d[1::2, ::3]
    yield "column", base2d[:, 7:8]
    yield "transpose_slice", base2d[2:-1, 4:].T


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_copy_views(hip, dtype):
    base = inputs(9, 300 * 517, dtype).reshape(300, 517)
    for name, view in views_of(base):
        assert_bitexact(strided_copy(hip, base, view, dtype), ref.strided_copy(view), name)
    base3 = inputs(10, 6 * 70 * 33, dtype).reshape(6, 70, 33)
    for perm in [(0, 2, 1), (2, 1, 0), (1, 0, 2), (2, 0, 1)]:
        view = base3.transpose(perm)
        assert_bitexact(strided_copy(hip, base3, view, dtype), ref.strided_copy(view), str(perm))
    bias = inputs(11, 33, dtype)
    expanded = np.broadcast_to(bias, (5, 7, 33))
    assert_bitexact(strided_copy(hip, bias, expanded, dtype), ref.strided_copy(expanded), "expand")


def strided_binary(hip, left_base, left_view, right_base, right_view, op, dtype):
    shape = np.broadcast_shapes(left_view.shape, right_view.shape)
    lv = np.broadcast_to(left_view, shape)
    rv = np.broadcast_to(right_view, shape)
    item = np.dtype(dtype).itemsize

    def geometry(base, view):
        offset = (view.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // item
        return [s // item for s in view.strides], offset

    ls, lo = geometry(left_base, lv)
    rs, ro = geometry(right_base, rv)
    check_span(left_base, shape, ls, lo)
    check_span(right_base, shape, rs, ro)
    dl, dr = dev(hip, left_base), dev(hip, right_base)
    out = out_buf(hip, shape, dtype)
    hip.call("spar_hip_launch_strided_binary", out.ptr, dl.ptr, hip.u64_array(ls), lo, dr.ptr,
             hip.u64_array(rs), ro, len(shape), hip.u64_array(shape), tag(dtype),
             hip.BINARY_OPS[op], 0)
    return out.to_numpy(dtype, shape), ref.binary(lv, rv, op)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("op", ["add", "subtract", "multiply", "divide", "less"])
def test_strided_binary_broadcasts(hip, dtype, op):
    x = inputs(12, 4 * 64 * 96, dtype).reshape(4, 64, 96)
    bias = inputs(13, 96, dtype)
    scale = inputs(14, 4 * 96, dtype).reshape(4, 1, 96)
    column = inputs(15, 4 * 64, dtype).reshape(4, 64, 1)
    one = inputs(16, 1, dtype)
    for name, rb, rv in [("bias", bias, bias), ("scale", scale, scale), ("column", column, column),
                         ("scalar", one, one)]:
        got, want = strided_binary(hip, x, x, rb, rv, op, dtype)
        assert_bitexact(got, want, f"x {op} {name}")
        got, want = strided_binary(hip, rb, rv, x, x, op, dtype)
        assert_bitexact(got, want, f"{name} {op} x")


def random_binary_operand(rng, shape, dtype, seed):
    """A view that broadcasts to `shape`: leading axes sometimes dropped, some
    axes of extent 1, stored in a random axis order inside a larger base and
    narrowed at random offsets."""
    lead = int(rng.integers(0, len(shape))) if rng.random() < 0.3 else 0
    vshape = [1 if rng.random() < 0.25 else e for e in shape[lead:]]
    order = [int(a) for a in rng.permutation(len(vshape))]
    stored = [vshape[a] for a in order]
    base_shape = [e + int(rng.integers(0, 3)) for e in stored]
    base = inputs(seed, int(np.prod(base_shape)), dtype).reshape(base_shape)
    starts = [int(rng.integers(0, b - e + 1)) for b, e in zip(base_shape, stored)]
    window = base[tuple(slice(s0, s0 + e) for s0, e in zip(starts, stored))]
    return base, window.transpose(np.argsort(order))


@pytest.mark.parametrize("dtype", DTYPES)
def test_random_strided_binary(hip, dtype):
    """Every binary op over 50 random pairs of broadcasting views (rank 1-4,
    permuted, narrowed, extent-1 and missing axes) against the oracle, bit for
    bit, with IEEE special values among the inputs."""
    rng = np.random.default_rng(92 if dtype == F32 else 93)
    ops = sorted(hip.BINARY_OPS)
    for case in range(50):
        rank = int(rng.integers(1, 5))
        while True:
            shape = [int(rng.choice([1, 2, 3, 7, 16, 33, 64, 100, 130, 256])) for _ in range(rank)]
            if int(np.prod(shape)) <= (2 << 20):
                break
        lb, lv = random_binary_operand(rng, shape, dtype, 2000 + 2 * case)
        rb, rv = random_binary_operand(rng, shape, dtype, 2001 + 2 * case)
        op = ops[int(rng.integers(0, len(ops)))]
        got, want = strided_binary(hip, lb, lv, rb, rv, op, dtype)
        assert_bitexact(got, want, f"case {case}: {list(lv.shape)} {op} {list(rv.shape)}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_binary_views(hip, dtype):
    base = inputs(17, 200 * 130, dtype).reshape(200, 130)
    other = inputs(18, 130 * 200, dtype).reshape(130, 200)
    mu = inputs(19, 130, dtype).reshape(130, 1)
    cases = [
        ("transpose-contig", base, base.T, other, other),
        ("contig-transpose", other, other, base, base.T),
        ("transpose-column", base, base.T, mu, mu),
        ("slice-slice", base, base[10:140, 3:103], base, base[50:180, 20:120]),
    ]
    for name, lb, lv, rb, rv in cases:
        got, want = strided_binary(hip, lb, lv, rb, rv, "subtract", dtype)
        assert_bitexact(got, want, name)


@pytest.mark.parametrize("dtype", DTYPES)
def test_transposed_views_vector_tiles(hip, dtype):
    """Extents that are multiples of the vector width take the 16-byte tiled
    transpose: partial tiles, batch axes, offsets, two transposed operands,
    and a second operand read along q, broadcast along q, or gathered."""
    base = inputs(40, 200 * 132, dtype).reshape(200, 132)
    other = inputs(41, 132 * 200, dtype).reshape(132, 200)
    twin = inputs(42, 200 * 132, dtype).reshape(200, 132)
    mu = inputs(43, 132, dtype).reshape(132, 1)
    wide = inputs(44, 132 * 600, dtype).reshape(132, 600)
    cube = inputs(45, 5 * 64 * 36, dtype).reshape(5, 64, 36)
    cube2 = inputs(46, 5 * 36 * 64, dtype).reshape(5, 36, 64)
    binary_cases = [
        ("T - contiguous", base, base.T, other, other),
        ("T - T", base, base.T, twin, twin.T),
        ("T - column", base, base.T, mu, mu),
        ("T - gathered", base, base.T, wide, wide[:, ::3]),
        ("contiguous - T", other, other, base, base.T),
        ("offset T", base, base[4:196, 8:132].T, other, other[8:132, 4:196]),
        ("unaligned offset T", base, base[1:197, 3:131].T, other, other[3:131, 1:197]),
        ("batched T", cube, cube.transpose(0, 2, 1), cube2, cube2),
        ("batch-outer T", cube, cube.transpose(2, 0, 1), cube, cube.transpose(2, 0, 1)),
    ]
    for name, lb, lv, rb, rv in binary_cases:
        got, want = strided_binary(hip, lb, lv, rb, rv, "subtract", dtype)
        assert_bitexact(got, want, name)
    # Each view is passed with the array it was taken from (offsets are
    # measured from that array's first element).
    for name, owner, view in [("T", base, base.T), ("offset T", base, base[4:196, 8:132].T),
                              ("batched T", cube, cube.transpose(0, 2, 1)),
                              ("perm", cube, cube.transpose(2, 0, 1)),
                              ("perm2", cube, cube.transpose(1, 2, 0))]:
        assert_bitexact(strided_copy(hip, owner, view, dtype), ref.strided_copy(view),
                        f"copy {name}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_transposed_tiles_walked_by_resident_workgroups(hip, dtype):
    """More tiles than resident workgroups (about 512 with one transposed
    operand, 256 with two): each workgroup walks several tiles and loads the
    next one while storing the current, across partial edge tiles and
    batch axes."""
    base = inputs(47, 2600 * 4000, dtype).reshape(2600, 4000)
    twin = inputs(48, 2600 * 4000, dtype).reshape(2600, 4000)
    mu = inputs(49, 4000, dtype).reshape(4000, 1)
    cube = inputs(50, 24 * 520 * 300, dtype).reshape(24, 520, 300)
    cube2 = inputs(51, 24 * 520 * 300, dtype).reshape(24, 520, 300)
    for name, lb, lv, rb, rv in [
        ("T - column", base, base.T, mu, mu),
        ("T - T", base, base.T, twin, twin.T),
        ("batched T - T", cube, cube.transpose(0, 2, 1), cube2, cube2.transpose(0, 2, 1)),
    ]:
        got, want = strided_binary(hip, lb, lv, rb, rv, "subtract", dtype)
        assert_bitexact(got, want, name)
    assert_bitexact(strided_copy(hip, base, base.T, dtype), ref.strided_copy(base.T), "copy T")


def test_strided_binary_odd_inner_extent(hip):
    # inner extent not a multiple of 4: row-vector path must not be taken
    x = inputs(20, 33 * 37, F32).reshape(33, 37)
    bias = inputs(21, 37, F32)
    got, want = strided_binary(hip, x, x, bias, bias, "add", F32)
    assert_bitexact(got, want, "odd inner")


# ------------------------------------------------------------ reductions

def axis_reduce(hip, base, view, axes, op, dtype):
    item = np.dtype(dtype).itemsize
    offset = (view.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // item
    strides = [s // item for s in view.strides]
    check_span(base, view.shape, strides, offset)
    mask = 0
    for a in axes:
        mask |= 1 << a
    kept = [d for i, d in enumerate(view.shape) if i not in axes]
    out_dtype = np.int64 if op == "argmax" else dtype
    out = out_buf(hip, kept, out_dtype)
    opcode = {"sum": hip.SUM, "mean": hip.MEAN, "max": hip.MAX, "argmax": hip.ARGMAX}[op]
    hip.call("spar_hip_launch_axis_reduction", out.ptr, dev(hip, base).ptr, view.ndim,
             hip.u64_array(view.shape), hip.u64_array(strides), offset, mask, tag(dtype), opcode, 0)
    return out.to_numpy(out_dtype, kept)


def check_axis(hip, base, view, axes, dtype, name):
    n = int(np.prod([view.shape[a] for a in axes]))
    s = ref.axis_sum(view, axes)
    norm = np.sqrt(ref.axis_sum((view.astype(np.float64) ** 2), axes))
    assert_red(axis_reduce(hip, base, view, axes, "sum", dtype), s, n, norm, f"{name} sum")
    mean_ref = ref.scalar(s, "divide", float(n)).reshape(s.shape) if s.ndim else s / dtype(n)
    assert_red(axis_reduce(hip, base, view, axes, "mean", dtype), mean_ref, n, norm / n,
               f"{name} mean")
    mx, am = ref.axis_max(view, axes)
    assert_bitexact(axis_reduce(hip, base, view, axes, "max", dtype), mx, f"{name} max")
    assert_bitexact(axis_reduce(hip, base, view, axes, "argmax", dtype), am, f"{name} argmax")


@pytest.mark.parametrize("dtype", DTYPES)
def test_axis_reductions_2d(hip, dtype):
    base = inputs(22, 512 * 1536, dtype, with_specials=False).reshape(512, 1536)
    for axes in ([0], [1], [0, 1]):
        check_axis(hip, base, base, axes, dtype, f"contig {axes}")
        check_axis(hip, base, base.T, axes, dtype, f"transposed {axes}")
    sliced = base[7:300, 8:1032]
    for axes in ([0], [1]):
        check_axis(hip, base, sliced, axes, dtype, f"sliced {axes}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_axis_reductions_3d(hip, dtype):
    base = inputs(23, 6 * 40 * 260, dtype, with_specials=False).reshape(6, 40, 260)
    for axes in ([0], [1], [2], [0, 1], [0, 2], [1, 2], [0, 1, 2]):
        check_axis(hip, base, base, axes, dtype, f"3d {axes}")
    perm = base.transpose(2, 0, 1)
    for axes in ([0], [2], [1, 2]):
        check_axis(hip, base, perm, axes, dtype, f"3d perm {axes}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 2, 3, 7, 16, 32, 33])
def test_short_row_reductions_exact(hip, dtype, n):
    """Rows of at most 32 contiguous elements take one lane per row, scanning
    in index order: sum, mean, max and argmax equal the oracle's in-order
    loops bit for bit (rows of 33 take the workgroup kernel: sum and mean
    within red(n)).  Rows hold NaNs, infinities, all -inf rows and ties; the
    rows are read in place from a block of a wider tensor and from a
    permuted view whose reduced axis is the contiguous one."""
    rows = 5000
    rng = np.random.default_rng(n)
    wide = np.round(rng.standard_normal((rows, n + 5)) * 4).astype(dtype) / dtype(4)
    wide[7, :] = -np.inf
    wide[11, min(2, n - 1)] = np.nan
    wide[13, 0] = np.inf
    wide[17, n // 2] = np.nan
    wide[17, n - 1] = np.inf
    block = wide[:, 2:2 + n]
    cube = np.ascontiguousarray(wide[: 4000].reshape(40, 100, n + 5)[:, :, :n])
    views = [(wide, block, [1], "block"), (cube, cube.transpose(1, 0, 2), [2], "permuted")]
    for base, view, axes, name in views:
        what = f"short rows n={n} {name}"
        s = ref.axis_sum(view, axes)
        mean_ref = ref.scalar(s, "divide", float(n))
        if n <= 32:
            assert_bitexact(axis_reduce(hip, base, view, axes, "sum", dtype), s, what + " sum")
            assert_bitexact(axis_reduce(hip, base, view, axes, "mean", dtype), mean_ref,
                            what + " mean")
        else:
            norm = np.sqrt(ref.axis_sum((view.astype(np.float64) ** 2), axes))
            assert_red(axis_reduce(hip, base, view, axes, "sum", dtype), s, n, norm, what)
        mx, am = ref.axis_max(view, axes)
        assert_bitexact(axis_reduce(hip, base, view, axes, "max", dtype), mx, what + " max")
        assert_bitexact(axis_reduce(hip, base, view, axes, "argmax", dtype), am, what + " argmax")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,axes", [((300, 2048), [0]), ((3, 200, 1100), [1]),
                                        ((2, 70, 4096), [0, 1]), ((5000, 1024), [0])])
def test_column_reductions_wide_rows(hip, dtype, shape, axes):
    """Rows of >= 256 vectors take the wave-per-column-range kernel; values
    are quantised so that maxima tie, and NaNs sit in some columns."""
    size = int(np.prod(shape))
    base = np.round(inputs(28, size, dtype, with_specials=False) * 8) / 8
    base = base.astype(dtype).reshape(shape)
    check_axis(hip, base, base, axes, dtype, f"wide {shape} {axes}")
    spiked = base.copy()
    flat = spiked.reshape(-1, shape[-1])
    flat[flat.shape[0] // 3, 5] = np.nan
    flat[flat.shape[0] // 2, 5] = np.nan
    flat[7, shape[-1] - 1] = np.inf
    spiked[..., 9] = -np.inf  # a column of -inf: argmax is its first row
    mx, am = ref.axis_max(spiked, axes)
    assert_bitexact(axis_reduce(hip, spiked, spiked, axes, "max", dtype), mx, "wide max nan")
    assert_bitexact(axis_reduce(hip, spiked, spiked, axes, "argmax", dtype), am, "wide argmax nan")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,axes", [((96, 8192), [0]), ((8, 8192), [1]), ((3, 40, 4096), [1])])
def test_max_argmax_nan_rescan(hip, dtype, shape, axes):
    """The scans compare NaN-free data with one ordered compare and rescan
    exactly the lanes that saw a NaN: NaNs (the first one wins), ties, signed
    zeros and -inf columns on the 4-group column path and the row path."""
    size = int(np.prod(shape))
    x = (np.round(inputs(31, size, dtype, with_specials=False) * 4) / 4).astype(dtype).reshape(shape)
    flat = x.reshape(-1, shape[-1])
    r = flat.shape[0]
    flat[r // 5, 100] = np.nan
    flat[r // 2, 100] = np.nan
    flat[r - 1, 4097 % shape[-1]] = np.nan
    flat[:, 7] = -0.0
    flat[r // 3, 7] = 0.0
    flat[:, 8] = -np.inf
    flat[2, 9] = np.inf
    flat[r - 1, 9] = np.inf
    for v in range(8):  # one NaN per 4-element group of a lane, in different rows
        flat[(v * 7) % r, 2048 + 64 * v] = np.nan
    mx, am = ref.axis_max(x, axes)
    assert_bitexact(axis_reduce(hip, x, x, axes, "max", dtype), mx, f"nan rescan max {shape}")
    assert_bitexact(axis_reduce(hip, x, x, axes, "argmax", dtype), am, f"nan rescan argmax {shape}")


STRIP_CASES = [
    # (dtype, base shape, view slices, reduced axes): max/argmax over a
    # contiguous kept axis wide enough for one 128-byte strip per CU
    (F32, (1000, 8192), None, [0]),
    (F32, (300, 8200), None, [0]),                                 # partial last strip
    (F64, (600, 4096), None, [0]),
    (F32, (2, 300, 8192), None, [1]),                              # two outer indices
    (F32, (400, 8208), (slice(3, 397), slice(8, 8200)), [0]),      # offset, padded rows
]


@pytest.mark.parametrize("case", range(len(STRIP_CASES)))
def test_max_argmax_column_strips(hip, case):
    """The one-pass strip kernel: lanes scan rows 32 apart, so ties, signed
    zeros, -inf columns and NaNs (first one wins) must resolve across lanes;
    a NaN in the tail rows and NaNs in several lanes of one column force the
    exact rescan."""
    dtype, shape, window, axes = STRIP_CASES[case]
    size = int(np.prod(shape))
    base = (np.round(inputs(34 + case, size, dtype, with_specials=False) * 4) / 4).astype(dtype)
    base = base.reshape(shape)
    view = base if window is None else base[window]
    flat = view if view.ndim == 2 else view[1]  # a view into base: writes reach it
    n = flat.shape[0]
    flat[:, 7] = -0.0
    flat[33, 7] = 0.0            # +0 in another lane after -0: -0 at row 0 wins
    flat[:, 8] = -np.inf         # all -inf: row 0
    flat[2, 9] = np.inf
    flat[n - 1, 9] = np.inf
    flat[n // 5, 100] = np.nan   # two NaNs in different lanes: the first wins
    flat[n // 2, 100] = np.nan
    flat[n - 3, 101] = np.nan    # in the tail rows
    flat[:, 102] = 1.0           # every row ties: row 0
    flat[40, 103] = 3.0          # ties between two lanes: row 40 before row 71
    flat[71, 103] = 3.0
    mx, am = ref.axis_max(view, axes)
    assert_bitexact(axis_reduce(hip, base, view, axes, "max", dtype), mx, f"strip max {case}")
    assert_bitexact(axis_reduce(hip, base, view, axes, "argmax", dtype), am, f"strip argmax {case}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows", [4096, 2048, 2400, 1024, 600, 160, 128])
def test_column_combine_split_counts(hip, dtype, rows):
    """Sum, mean, max and argmax over axis 0 of [rows, 4096]: the column pass
    takes one workgroup per CU, so it splits the rows into min(CUs, rows / 16)
    ranges (float32 on a 256-CU device: 256, 128, 150, 64, 36, 10 and 8), and
    the combine meets every batch form: 16 x 16, 16 x 8, 4 x 8 and 1 x 8
    without bounds tests, and tested loads for the other counts.  Values are
    quantised so that maxima tie across splits; one column holds NaNs and one
    is all -inf."""
    cols = 4096
    x = np.round(inputs(36, rows * cols, dtype, with_specials=False) * 8) / 8
    x = x.astype(dtype).reshape(rows, cols)
    x[rows // 3, 11] = np.nan
    x[rows - 1, 11] = np.nan
    x[:, 12] = -np.inf
    x[:, 13] = 0.5
    check_axis(hip, x, x, [0], dtype, f"split counts [{rows}, {cols}]")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("outer,rows", [(2, 2048), (3, 1400), (5, 512)])
def test_column_combine_outer_indices(hip, dtype, outer, rows):
    """The same reductions over axis 1 of [outer, rows, 4096]: every outer
    index has its own splits (float32 on a 256-CU device: 128, 83 and 32 per
    outer index), so the combine's outer-index arithmetic meets exact and
    tested batches alike."""
    cols = 4096
    x = np.round(inputs(37 + outer, outer * rows * cols, dtype, with_specials=False) * 8) / 8
    x = x.astype(dtype).reshape(outer, rows, cols)
    x[outer - 1, rows // 2, 17] = np.nan
    x[0, :, 18] = -np.inf
    check_axis(hip, x, x, [1], dtype, f"outer {outer} x [{rows}, {cols}]")


def random_reduction_case(rng):
    """A random view of a random base and a random set of reduced axes: rank 1
    to 4, extents 1 to 300 (views up to 4 M elements), the view's axes
    permuted and each narrowed at a random offset."""
    rank = int(rng.integers(1, 5))
    while True:
        shape = [int(rng.choice([1, 2, 3, 7, 16, 33, 64, 100, 256, 300])) for _ in range(rank)]
        if int(np.prod(shape)) <= (4 << 20):
            break
    base_shape = [e + int(rng.integers(0, 3)) for e in shape]
    starts = [int(rng.integers(0, b - e + 1)) for b, e in zip(base_shape, shape)]
    order = [int(a) for a in rng.permutation(rank)]
    count = int(rng.integers(1, rank + 1))
    axes = sorted(int(a) for a in rng.choice(rank, count, replace=False))
    return base_shape, starts, shape, order, axes


@pytest.mark.parametrize("dtype", DTYPES)
def test_random_axis_reductions(hip, dtype):
    """Sum, mean, max and argmax of 60 random views and axis sets against the
    oracle: every planner path (row, column, column strip, interleaved, narrow
    and generic kernels, with and without splits) on layouts nobody chose.
    Values are quantised so that maxima tie."""
    rng = np.random.default_rng(90 if dtype == F32 else 91)
    for case in range(60):
        base_shape, starts, shape, order, axes = random_reduction_case(rng)
        size = int(np.prod(base_shape))
        base = (np.round(inputs(1000 + case, size, dtype, with_specials=False) * 4) / 4)
        base = base.astype(dtype).reshape(base_shape)
        window = tuple(slice(s0, s0 + e) for s0, e in zip(starts, shape))
        view = base[window].transpose(order)
        check_axis(hip, base, view, axes, dtype,
                   f"case {case}: base {base_shape} view {list(view.shape)} axes {axes}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows", [8192, 700])
def test_column_max_value_only_across_splits(hip, dtype, rows):
    """A max without argmax over wide rows keeps no indices: ties between
    splits (signed zeros, NaN payloads) must still resolve to the first
    occurrence, ordered by split."""
    cols = 4096
    x = -np.abs(inputs(33, rows * cols, dtype, with_specials=False)).reshape(rows, cols) - 1
    x[rows - 1, 0] = 0.0      # +0 last, -0 first: -0
    x[3, 0] = -0.0
    x[2, 1] = 0.0             # +0 first, -0 later: +0
    x[rows - 2, 1] = -0.0
    x[:, 2] = 5.0             # every row ties
    x[:, 3] = -np.inf
    quiet = np.array([0x7FC00001, 0x7FC00002], dtype=np.uint32) if dtype == F32 else \
        np.array([0x7FF8000000000001, 0x7FF8000000000002], dtype=np.uint64)
    nans = quiet.view(dtype)
    x[rows // 2, 4] = nans[1]  # later NaN
    x[rows // 4, 4] = nans[0]  # first NaN: its payload is the result
    x[rows - 1, 5] = nans[1]
    mx, _ = ref.axis_max(x, [0])
    got = axis_reduce(hip, x, x, [0], "max", dtype)
    assert_bitexact(got, mx, f"value-only max {rows}")
    assert np.signbit(got[0]) and not np.signbit(got[1])
    assert got[4:5].view(quiet.dtype)[0] == quiet[0]
    assert np.isnan(got[5]) and got[2] == 5.0 and got[3] == -np.inf


@pytest.mark.parametrize("dtype", DTYPES)
def test_max_argmax_negative_infinity_runs(hip, dtype):
    """Rows long enough to be split over blocks, made of -inf runs: the answer
    is the first -inf unless a NaN or a finite value appears later."""
    cols = 200000
    x = inputs(29, 4 * cols, dtype, with_specials=False).reshape(4, cols)
    x[1:] = -np.inf
    x[2, 150000] = np.nan
    x[3, cols - 1] = 1.0
    mx, am = ref.axis_max(x, [1])
    assert list(am) == [int(np.argmax(x[0])), 0, 150000, cols - 1]
    assert_bitexact(axis_reduce(hip, x, x, [1], "max", dtype), mx, "-inf rows max")
    assert_bitexact(axis_reduce(hip, x, x, [1], "argmax", dtype), am, "-inf rows argmax")
    flat = np.full(1 << 20, -np.inf, dtype=dtype)
    out = out_buf(hip, (1,), np.int64)
    hip.call("spar_hip_launch_reduction", out.ptr, dev(hip, flat).ptr, flat.size, tag(dtype),
             hip.ARGMAX, 0)
    assert out.to_numpy(np.int64, (1,))[0] == 0
    hip.call("spar_hip_launch_reduction", out.ptr, dev(hip, flat).ptr, flat.size, tag(dtype),
             hip.MAX, 0)
    assert out.to_numpy(dtype, (1,))[0] == -np.inf


def test_max_argmax_ties_nan_signed_zero(hip):
    rows = np.array([
        [1.0, 3.0, 3.0, 2.0],
        [-0.0, 0.0, -1.0, 0.0],
        [0.0, -0.0, -0.0, -2.0],
        [1.0, np.nan, 5.0, np.nan],
        [-np.inf, -np.inf, -np.inf, -np.inf],
        [np.inf, 1.0, np.inf, 0.0],
    ], dtype=F32)
    got = axis_reduce(hip, rows, rows, [1], "max", F32)
    want, want_idx = ref.axis_max(rows, [1])
    assert_bitexact(got, want, "max ties")
    assert_bitexact(axis_reduce(hip, rows, rows, [1], "argmax", F32), want_idx, "argmax ties")
    assert list(want_idx) == [1, 0, 0, 1, 0, 0]
    assert np.signbit(got[1]) and not np.signbit(got[2])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1 << 20, 4 * (5 * 512 * 256 + 77)])
def test_full_max_argmax_special(hip, dtype, n):
    """Full max and argmax of long rows (the interleaved scan, whose lanes
    take vectors a grid apart): a maximum repeated in other workgroups and
    lanes, NaNs (the first wins), a -0 maximum ahead of a +0, +inf twice and
    a -inf row with one late NaN, each against the oracle's in-order scan."""
    rng = np.random.default_rng(n)
    cases = []
    x = rng.uniform(-1, 1, n).astype(dtype)
    x[[n // 7, n // 3, n - 5]] = dtype(2.5)           # repeated maximum
    cases.append(x)
    x = rng.uniform(-1, 1, n).astype(dtype)
    x[[n // 2, n // 9]] = np.nan                      # two NaNs: index n // 9 first
    cases.append(x)
    x = np.full(n, -1.0, dtype=dtype)
    x[1001] = -0.0
    x[n - 1000] = 0.0                                 # -0 first: max is -0 at 1001
    cases.append(x)
    x = rng.uniform(-1, 1, n).astype(dtype)
    x[[4099, 3 * n // 4]] = np.inf
    cases.append(x)
    x = np.full(n, -np.inf, dtype=dtype)
    x[n - 3] = np.nan
    cases.append(x)
    out = out_buf(hip, (1,), np.int64)
    for k, x in enumerate(cases):
        mx, am = ref.axis_max(x.reshape(1, n), [1])
        d = dev(hip, x)
        hip.call("spar_hip_launch_reduction", out.ptr, d.ptr, n, tag(dtype), hip.MAX, 0)
        assert_bitexact(out.to_numpy(dtype, (1,)), mx.reshape(1), f"full max case {k}")
        hip.call("spar_hip_launch_reduction", out.ptr, d.ptr, n, tag(dtype), hip.ARGMAX, 0)
        assert out.to_numpy(np.int64, (1,))[0] == int(am.reshape(-1)[0]), f"full argmax case {k}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 5, 1000, 1 << 16, 3 * (1 << 18) + 7, 1 << 20,
                               4 * (5 * 512 * 256 + 77), 1 << 25])
def test_full_reduction(hip, dtype, n):
    """Full sum, mean, max and argmax.  Long vector-aligned rows take the
    interleaved sum (several loop trips and a remainder for the middle
    sizes); the others the split scan."""
    x = (np.random.default_rng(24).random(n) * 2 - 1).astype(dtype)
    dx = dev(hip, x)
    out = out_buf(hip, (1,), np.int64)
    norm = float(np.sqrt(np.sum(x.astype(np.float64) ** 2)))
    for op, code in [("sum", hip.SUM), ("mean", hip.MEAN)]:
        hip.call("spar_hip_launch_reduction", out.ptr, dx.ptr, n, tag(dtype), code, 0)
        got = out.to_numpy(dtype, (1,))[0]
        want = ref.full_reduce(x, op)
        assert_red(got, want, n, norm / (n if op == "mean" else 1), f"full {op}")
    hip.call("spar_hip_launch_reduction", out.ptr, dx.ptr, n, tag(dtype), hip.MAX, 0)
    assert_bitexact(out.to_numpy(dtype, (1,)), np.array([ref.full_reduce(x, "max")]), "full max")
    hip.call("spar_hip_launch_reduction", out.ptr, dx.ptr, n, tag(dtype), hip.ARGMAX, 0)
    assert out.to_numpy(np.int64, (1,))[0] == int(np.argmax(x))


@pytest.mark.parametrize("dtype", DTYPES)
def test_row_reduction(hip, dtype):
    rows, cols = 77, 3000
    x = inputs(25, rows * cols, dtype, with_specials=False).reshape(rows, cols)
    out = out_buf(hip, (rows,), np.int64)
    dx = dev(hip, x)
    hip.call("spar_hip_launch_row_reduction", out.ptr, dx.ptr, rows, cols, tag(dtype), hip.SUM, 0)
    norm = np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=1))
    assert_red(out.to_numpy(dtype, (rows,)), ref.axis_sum(x, [1]), cols, norm, "row sum")
    hip.call("spar_hip_launch_row_reduction", out.ptr, dx.ptr, rows, cols, tag(dtype), hip.ARGMAX, 0)
    assert_bitexact(out.to_numpy(np.int64, (rows,)), ref.axis_max(x, [1])[1], "row argmax")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("gshape,oshape", [
    ((4, 64, 96), (96,)), ((4, 64, 96), (4, 1, 96)), ((4, 64, 96), (64, 1)),
    ((4, 64, 96), (1, 64, 96)), ((4, 64, 96), (4, 64, 96)), ((4, 64, 96), ()),
    ((3, 1, 5), (1, 5)), ((2048, 36), (36,)),
    ((512, 4096), ()),   # a long full reduction: the interleaved scan, sum and product
])
def test_broadcast_reduce_and_product(hip, dtype, gshape, oshape):
    g = inputs(26, int(np.prod(gshape)), dtype, with_specials=False).reshape(gshape)
    f = inputs(27, int(np.prod(gshape)), dtype, with_specials=False).reshape(gshape)
    out = out_buf(hip, oshape, dtype)
    n = max(int(np.prod(gshape)) // max(int(np.prod(oshape)), 1), 1)
    want = ref.reduce_gradient(g, oshape)
    norm = np.sqrt(ref.reduce_gradient(g.astype(np.float64) ** 2, oshape))
    hip.call("spar_hip_launch_broadcast_reduce", out.ptr, dev(hip, g).ptr, len(gshape),
             hip.u64_array(gshape), len(oshape), hip.u64_array(oshape), hip.u64_array([0] * 8),
             g.size, tag(dtype), 0)
    assert_red(out.to_numpy(dtype, oshape), want, n, norm, f"reduce {gshape}->{oshape}")
    # multiply backward: reduce_gradient_to_shape(multiply(g, f)) in one pass
    product = ref.binary(g, f, "multiply")
    want = ref.reduce_gradient(product, oshape)
    norm = np.sqrt(ref.reduce_gradient(product.astype(np.float64) ** 2, oshape))
    hip.call("spar_hip_launch_multiply_reduce", out.ptr, dev(hip, g).ptr, dev(hip, f).ptr,
             len(gshape), hip.u64_array(gshape), len(oshape), hip.u64_array(oshape), g.size,
             tag(dtype), 0)
    assert_red(out.to_numpy(dtype, oshape), want, n, norm, f"multiply_reduce {gshape}->{oshape}")


# --------------------------------------------------------------- softmax

def softmax_device(hip, x, outer, extent, inner, log, dtype):
    out = out_buf(hip, x.shape, dtype)
    undefined = out_buf(hip, (outer * inner,), np.int32)
    hip.call("spar_hip_launch_probability_forward", out.ptr, undefined.ptr, dev(hip, x).ptr, outer,
             extent, inner, tag(dtype), int(log), 0)
    return out.to_numpy(dtype, x.shape), undefined.to_numpy(np.int32, (outer * inner,))


def softmax_tolerance_check(got, want, extent, dtype, what):
    """p = e / S: exp within 2 ulp, S within red(extent), one more rounding:
    |dp| <= (4 eps + 1e-6 sqrt(extent)) |p| (+ tiny for underflowed p)."""
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    eps = np.finfo(dtype).eps
    bound = (4 * eps + 1e-6 * np.sqrt(extent)) * np.abs(want) + np.finfo(dtype).tiny
    ok = gn | (got == want) | (np.abs(got.astype(np.float64) - want) <= bound)
    assert ok.all(), f"{what}: {(~ok).sum()} elements out of tolerance"


def log_softmax_tolerance_check(got, want, extent, dtype, what):
    """lp = (x - m) - log S: x - m is exact on both sides; log S differs by
    S's relative difference (red) plus log's rounding; one final rounding:
    |dlp| <= 1e-6 sqrt(extent) + 4 eps (|lp| + log(extent) + 1)."""
    eps = np.finfo(dtype).eps
    finite = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want)), what
    assert np.array_equal(got[~finite & ~np.isnan(want)], want[~finite & ~np.isnan(want)]), what
    err = np.abs(got[finite].astype(np.float64) - want[finite])
    bound = 1e-6 * np.sqrt(extent) + 4 * eps * (np.abs(want[finite]) + np.log(extent) + 1)
    assert np.all(err <= bound), f"{what}: max err {err.max()}"


def softmax_backward_bound(g, y, extent, dtype, log):
    """softmax: dx = y (g - dot), |d dot| <= red(extent) with scale ||g||_2
    (|y| <= 1), so |d dx| <= 1e-6 sqrt(n) ||g|| |y| + 4 eps (|dx| + |y| (|g| + max|g|)).
    log-softmax: dx = g - exp(lp) s, |d s| <= 1e-6 sqrt(n) max(|s|, ||g||),
    exp within 2 ulp: |d dx| <= e (1e-6 sqrt(n) max(|s|, ||g||) + 3 eps |s|) + 4 eps (|dx| + |g|)."""
    eps = np.finfo(dtype).eps
    g64 = g.astype(np.float64)
    norm = np.sqrt(np.sum(g64 ** 2, axis=-1, keepdims=True))
    if not log:
        dot = np.sum(g64 * y, axis=-1, keepdims=True)
        dx = y * (g64 - dot)
        bound = 1e-6 * np.sqrt(extent) * norm * np.abs(y) + 4 * eps * (
            np.abs(dx) + np.abs(y) * (np.abs(g64) + np.abs(g64).max(axis=-1, keepdims=True)))
    else:
        e = np.exp(y.astype(np.float64))
        total = np.sum(g64, axis=-1, keepdims=True)
        dx = g64 - e * total
        bound = e * (1e-6 * np.sqrt(extent) * np.maximum(np.abs(total), norm)
                     + 3 * eps * np.abs(total)) + 4 * eps * (np.abs(dx) + np.abs(g64))
    return bound + np.finfo(dtype).tiny


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,extent", [(3, 1), (5, 7), (40, 200), (64, 1000), (16, 1024),
                                         (8, 2000), (8, 4096), (4, 6000), (4, 8192), (4, 12000),
                                         (2, 16384), (2, 32000), (2, 32768), (2, 32770),
                                         (1, 40000)])
def test_softmax_rows(hip, dtype, rows, extent):
    x = (inputs(28, rows * extent, dtype, with_specials=False) * dtype(np.sqrt(2))).reshape(rows, extent)
    got, und = softmax_device(hip, x, rows, extent, 1, False, dtype)
    want, und_ref = ref.softmax_axis(x, 1)
    softmax_tolerance_check(got, want, extent, dtype, f"softmax {rows}x{extent}")
    assert np.array_equal(und, und_ref.astype(np.int32))
    lgot, _ = softmax_device(hip, x, rows, extent, 1, True, dtype)
    lwant, _ = ref.log_softmax(x, 1)
    log_softmax_tolerance_check(lgot, lwant, extent, dtype, f"log_softmax {rows}x{extent}")

    g = inputs(29, rows * extent, dtype, with_specials=False).reshape(rows, extent)
    dund = dev(hip, und_ref.astype(np.int32))
    for log, saved, back in [(False, want, ref.softmax_axis_backward(g, want, und_ref, 1)),
                             (True, lwant, ref.log_softmax_backward(g, lwant, und_ref, 1))]:
        out = out_buf(hip, x.shape, dtype)
        hip.call("spar_hip_launch_probability_backward", out.ptr, dev(hip, g).ptr,
                 dev(hip, saved).ptr, dund.ptr, rows, extent, 1, tag(dtype), int(log), 0)
        got_b = out.to_numpy(dtype, x.shape)
        err = np.abs(got_b.astype(np.float64) - back)
        bound = softmax_backward_bound(g, saved, extent, dtype, log)
        assert np.all(err <= bound), f"backward log={log} worst {(err / bound).max()}x bound"


@pytest.mark.parametrize("dtype", DTYPES)
def test_softmax_special_slices(hip, dtype):
    inf, nan = np.inf, np.nan
    x = np.array([
        [1.0, 2.0, 3.0, 4.0],
        [nan, 1.0, 2.0, 3.0],
        [-inf, -inf, -inf, -inf],
        [inf, 1.0, inf, -inf],
        [inf, 0.0, 0.0, 0.0],
        [-inf, 0.0, -inf, 1.0],
        [-0.0, 0.0, -inf, -inf],
    ], dtype=dtype)
    rows, extent = x.shape
    for log in (False, True):
        got, und = softmax_device(hip, x, rows, extent, 1, log, dtype)
        want, und_ref = (ref.log_softmax(x, 1) if log else ref.softmax_axis(x, 1))
        assert np.array_equal(und, und_ref.astype(np.int32))
        assert_ulp(got, want, 2, f"special log={log}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("extent", [1000, 12000, 32000, 32768, 32770])
def test_softmax_special_long_rows(hip, dtype, extent):
    """Undefined and +inf rows at every register-row shape, full and partial
    (their slow path reloads the row), beside rows of equal values."""
    inf, nan = np.inf, np.nan
    x = np.zeros((8, extent), dtype=dtype)
    x[0, extent // 3] = nan
    x[1, :] = -inf
    x[2, [5, extent - 2]] = inf
    x[2, 7] = -inf
    x[3, extent - 1] = inf
    x[4, :] = 2.5
    x[5, ::2] = -0.0
    x[6, :] = -inf
    x[6, extent // 2] = 1.0
    x[7, :] = 3.0
    x[7, extent - 1] = nan
    rows = x.shape[0]
    for log in (False, True):
        got, und = softmax_device(hip, x, rows, extent, 1, log, dtype)
        want, und_ref = (ref.log_softmax(x, 1) if log else ref.softmax_axis(x, 1))
        assert np.array_equal(und, und_ref.astype(np.int32))
        assert_ulp(got, want, 2, f"special long rows {extent} log={log}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("extent", [7, 1000, 32768])
def test_softmax_zero_maximum_bits(hip, dtype, extent):
    """Rows whose maximum is a signed zero, alone or beside the other zero
    (with -inf or very negative values elsewhere, so that S can be exactly
    1): the register-row forward takes the maximum by value, whichever zero
    it meets, and must give the oracle's first-occurrence results bit for
    bit, zero signs included."""
    inf = np.inf
    x = np.full((6, extent), -inf, dtype=dtype)
    x[0, 0] = -0.0
    x[1, :] = -200.0 if dtype == F32 else -1000.0  # exp underflows to +0
    x[1, extent - 1] = -0.0
    x[2, 1] = -0.0
    x[2, extent - 1] = 0.0
    x[3, 0] = 0.0
    x[3, extent // 2] = -0.0
    x[4, :] = -1e30
    x[4, 3] = -0.0
    x[5, 2] = 0.0
    rows = x.shape[0]
    for log in (False, True):
        got, und = softmax_device(hip, x, rows, extent, 1, log, dtype)
        want, und_ref = (ref.log_softmax(x, 1) if log else ref.softmax_axis(x, 1))
        assert not und_ref.any() and not und.any()
        bits = np.uint32 if dtype == F32 else np.uint64
        assert np.array_equal(got.view(bits), want.astype(dtype).view(bits)), \
            f"zero maximum rows, extent {extent} log={log}"


def test_softmax_rows_beyond_one_grid(hip):
    """More rows than one launch grid holds (2^20): the rows go out in
    several grids at shifted offsets."""
    rows, extent = (1 << 20) + 3, 4
    x = inputs(32, rows * extent, F32, with_specials=False).reshape(rows, extent)
    x[-1, 2] = np.nan
    got, und = softmax_device(hip, x, rows, extent, 1, False, F32)
    want, und_ref = ref.softmax_axis(x, 1)
    assert np.array_equal(und, und_ref.astype(np.int32))
    softmax_tolerance_check(got[:-1], want[:-1], extent, F32, "softmax beyond one grid")
    assert np.all(np.isnan(got[-1]))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,axis", [((6, 50, 33), 1), ((40, 9), 0), ((3, 4, 5, 6), 2)])
def test_softmax_inner_axis(hip, dtype, shape, axis):
    x = inputs(30, int(np.prod(shape)), dtype, with_specials=False).reshape(shape)
    outer = int(np.prod(shape[:axis]))
    inner = int(np.prod(shape[axis + 1:]))
    got, und = softmax_device(hip, x, outer, shape[axis], inner, False, dtype)
    want, und_ref = ref.softmax_axis(x, axis)
    softmax_tolerance_check(got, want, shape[axis], dtype, "inner-axis softmax")
    g = inputs(31, x.size, dtype, with_specials=False).reshape(shape)
    back = ref.softmax_axis_backward(g, want, und_ref, axis)
    out = out_buf(hip, shape, dtype)
    hip.call("spar_hip_launch_probability_backward", out.ptr, dev(hip, g).ptr, dev(hip, want).ptr,
             dev(hip, und_ref.astype(np.int32)).ptr, outer, shape[axis], inner, tag(dtype), 0, 0)
    err = np.abs(out.to_numpy(dtype, shape).astype(np.float64) - back)
    g_axis_last = np.moveaxis(g, axis, -1)
    y_axis_last = np.moveaxis(want, axis, -1)
    bound = np.moveaxis(softmax_backward_bound(g_axis_last, y_axis_last, shape[axis], dtype, False),
                        -1, axis)
    assert np.all(err <= bound)


@pytest.mark.parametrize("dtype", DTYPES)
def test_random_softmax_shapes(hip, dtype):
    """Softmax and log-softmax, forward and backward, over 30 random
    [outer, extent, inner] shapes (extents around the row kernels' register
    sizes and past the longest one, inner slices of 1 to 17) against the
    oracle within the derived bounds."""
    rng = np.random.default_rng(94 if dtype == F32 else 95)
    extents = [1, 2, 5, 63, 64, 65, 255, 256, 1000, 1024, 3000, 8193, 16385, 32769, 40000]
    for case in range(30):
        while True:
            outer = int(rng.integers(1, 200))
            extent = int(rng.choice(extents))
            inner = int(rng.choice([1, 1, 1, 2, 3, 17]))
            if outer * extent * inner <= (2 << 20):
                break
        shape = (outer, extent, inner)
        what = f"case {case}: {list(shape)}"
        x = (inputs(3000 + case, outer * extent * inner, dtype, with_specials=False)
             * dtype(2)).reshape(shape)
        g = inputs(4000 + case, x.size, dtype, with_specials=False).reshape(shape)
        for log in (False, True):
            got, und = softmax_device(hip, x, outer, extent, inner, log, dtype)
            if log:
                want, und_ref = ref.log_softmax(x, 1)
                log_softmax_tolerance_check(got, want, extent, dtype, what + " log fwd")
                back = ref.log_softmax_backward(g, want, und_ref, 1)
            else:
                want, und_ref = ref.softmax_axis(x, 1)
                softmax_tolerance_check(got, want, extent, dtype, what + " fwd")
                back = ref.softmax_axis_backward(g, want, und_ref, 1)
            assert np.array_equal(und, und_ref.astype(np.int32).ravel()), what
            out = out_buf(hip, shape, dtype)
            hip.call("spar_hip_launch_probability_backward", out.ptr, dev(hip, g).ptr,
                     dev(hip, want).ptr, dev(hip, und_ref.astype(np.int32)).ptr, outer, extent,
                     inner, tag(dtype), int(log), 0)
            err = np.abs(out.to_numpy(dtype, shape).astype(np.float64) - back)
            bound = np.moveaxis(softmax_backward_bound(np.moveaxis(g, 1, -1),
                                                       np.moveaxis(want, 1, -1), extent, dtype,
                                                       log), -1, 1)
            assert np.all(err <= bound), f"{what} backward log={log}"


# ---------------------------------------------------------------- random

@pytest.mark.parametrize("dtype", DTYPES)
def test_random_uniform_matches_host_generator(hip, dtype):
    n = 100001
    out = out_buf(hip, (n,), dtype)
    hip.call("spar_hip_random_uniform", out.ptr, n, tag(dtype), 1234, -1.0, 1.0, 0)
    want = ref.Random(1234).uniform((n,), dtype, -1.0, 1.0)
    assert_bitexact(out.to_numpy(dtype, (n,)), want, "uniform")


def test_random_normal_close_to_host_generator(hip):
    n = 100001
    out = out_buf(hip, (n,), F32)
    hip.call("spar_hip_random_normal", out.ptr, n, 0, 99, 0.0, 2.0, 0)
    want = ref.Random(99).normal((n,), F32, 0.0, 2.0)
    assert_ulp(out.to_numpy(F32, (n,)), want, 1, "normal")


# ----------------------------------------------------------- error paths

def test_status_codes_on_device(hip):
    st = hip.status_of("spar_hip_launch_binary", None, None, None, 0, 0, 0, 0)
    assert st.code == 0  # count 0: success without touching the device
    st = hip.status_of("spar_hip_launch_binary", None, None, None, 5, 0, 0, 0)
    assert st.code == 1
    st = hip.status_of("spar_hip_launch_unary", None, None, 0, 0, 0, 999)
    assert st.code == 0
    st = hip.status_of("spar_hip_synchronize", 999)
    assert st.code == 2
