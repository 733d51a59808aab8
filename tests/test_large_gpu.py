"""Counts past 2^31 elements: the launchers' 64-bit index paths.

The reference's launchers take uint64_t counts with grid-stride loops
(src/backend/cuda_kernels.cu:97-103, cuda_kernels.hpp:46-63); this backend
switches to 64-bit coordinates where a count or a row count passes
2^31 - 1.  One float32 tensor of 2^31 + 16 elements (8.6 GB) drives:

  * contiguous add (64-bit vector indices);
  * a broadcast add over [134217729, 16] + bias[16] (the generic strided
    kernel with 64-bit coordinate decoding: the row-vector paths take 32-bit
    rows only);
  * full sum and max, and argmax along the axis of [1, 2^31 + 16] with the
    maximum planted past 2^31 (a row split into segments below 2^31 whose
    partial indices are rebased in 64 bits);
  * a sum over the unit axis of [2^31 + 16, 1] (2^31 + 16 rows: the
    reduction's 64-bit row map).

Elementwise results are compared with the oracle on windows at the start,
across element 2^31 and at the end; the full sum within red(N) of a float64
sum of every element.  Before each launch the largest offset the launch can
touch is checked on the host against its buffer.
"""
import numpy as np
import pytest

from oracle import ops as ref
from tests.helpers import assert_bitexact, assert_red

pytestmark = pytest.mark.gpu

F32 = np.float32
N = (1 << 31) + 16
ROWS, COLS = N // 16, 16  # 134217729 x 16


def window(hip, buffer, start, count, dtype=F32, shape=None):
    item = np.dtype(dtype).itemsize
    assert 0 <= start and (start + count) * item <= buffer.nbytes, "window inside the buffer"
    out = np.empty(count, dtype)
    hip.call("spar_hip_copy_device_to_host", out.ctypes.data, buffer.address(start * item),
             count * item, 0)
    return out if shape is None else out.reshape(shape)


def largest_offset(shape, strides, offset=0):
    return offset + sum((d - 1) * s for d, s in zip(shape, strides) if d > 0)


@pytest.fixture(scope="module")
def big(hip):
    a = hip.DeviceBuffer(N * 4)
    b = hip.DeviceBuffer(N * 4)
    out = hip.DeviceBuffer(N * 4)
    hip.call("spar_hip_random_normal", a.ptr, N, hip.FLOAT32, 71, 0.0, 1.0, 0)
    hip.call("spar_hip_random_normal", b.ptr, N, hip.FLOAT32, 72, 0.0, 1.0, 0)
    hip.synchronize()
    yield a, b, out
    for buffer in (a, b, out):
        buffer.free()


# the last window holds elements 2^31 - 4080 to 2^31 + 15
WINDOWS = [(0, 4096), ((1 << 30) + 12345, 4096), (N - 4096, 4096)]


def test_contiguous_add_past_2_31(hip, big):
    a, b, out = big
    assert N * 4 <= min(a.nbytes, b.nbytes, out.nbytes)
    hip.call("spar_hip_launch_binary", out.ptr, a.ptr, b.ptr, N, hip.FLOAT32, hip.ADD, 0)
    for start, count in WINDOWS:
        want = ref.binary(window(hip, a, start, count), window(hip, b, start, count), "add")
        assert_bitexact(window(hip, out, start, count), want, f"add at {start}")


def test_broadcast_add_past_2_31(hip, big):
    a, _, out = big
    bias = np.random.default_rng(73).uniform(-0.1, 0.1, COLS).astype(F32)
    bias_dev = hip.DeviceBuffer.from_numpy(bias)
    shape = [ROWS, COLS]
    x_strides, bias_strides = [COLS, 1], [0, 1]
    assert largest_offset(shape, x_strides) < N and largest_offset(shape, bias_strides) < COLS
    u = hip.u64_array
    hip.call("spar_hip_launch_strided_binary", out.ptr, a.ptr, u(x_strides), 0, bias_dev.ptr,
             u(bias_strides), 0, 2, u(shape), hip.FLOAT32, hip.ADD, 0)
    for first_row, rows in ((0, 256), (ROWS - 256, 256)):  # the last rows hold element 2^31
        x = window(hip, a, first_row * COLS, rows * COLS, shape=(rows, COLS))
        got = window(hip, out, first_row * COLS, rows * COLS, shape=(rows, COLS))
        assert_bitexact(got, ref.binary(x, bias, "add"), f"broadcast add at row {first_row}")
    bias_dev.free()


def test_full_reductions_and_argmax_past_2_31(hip, big):
    a, _, _ = big
    planted = (1 << 31) + 5
    peak = np.array([100.0], F32)
    hip.call("spar_hip_copy_host_to_device", a.address(planted * 4), peak.ctypes.data, 4, 0)
    result = hip.DeviceBuffer(16)
    hip.call("spar_hip_launch_reduction", result.ptr, a.ptr, N, hip.FLOAT32, hip.MAX, 0)
    assert result.to_numpy(F32, (1,))[0] == F32(100.0)
    hip.call("spar_hip_launch_axis_reduction", result.ptr, a.ptr, 2, hip.u64_array([1, N]),
             hip.u64_array([N, 1]), 0, 1 << 1, hip.FLOAT32, hip.ARGMAX, 0)
    assert int(result.to_numpy(np.int64, (1,))[0]) == planted
    hip.call("spar_hip_launch_reduction", result.ptr, a.ptr, N, hip.FLOAT32, hip.SUM, 0)
    got = result.to_numpy(F32, (1,))
    want, squares = 0.0, 0.0
    for start in range(0, N, 1 << 27):  # float64 sums over 512 MiB windows
        values = window(hip, a, start, min(1 << 27, N - start)).astype(np.float64)
        want += float(np.sum(values))
        squares += float(np.sum(values * values))
    assert_red(got, np.array([want]), N, np.sqrt(squares), "full sum of 2^31 + 16")
    result.free()


def test_row_map_past_2_31_rows(hip, big):
    """A sum over the unit axis of [2^31 + 16, 1]: every output is its one
    element added to zero (the oracle's loop), 2^31 + 16 rows."""
    a, _, out = big
    hip.call("spar_hip_launch_axis_reduction", out.ptr, a.ptr, 2, hip.u64_array([N, 1]),
             hip.u64_array([1, 1]), 0, 1 << 1, hip.FLOAT32, hip.SUM, 0)
    for start, count in WINDOWS:
        x = window(hip, a, start, count, shape=(count, 1))
        assert_bitexact(window(hip, out, start, count), ref.axis_sum(x, [1]),
                        f"unit-axis sum at row {start}")
