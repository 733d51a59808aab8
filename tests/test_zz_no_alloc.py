"""spar_hip_launch_axis_reduction_no_alloc against spar_hip_launch_axis_reduction.

The no-allocation entry point runs the same plans and kernels with its
partial results in a fixed per-device workspace, so every output must equal
the allocating entry point's bit for bit (argmax indices included), and the
caching allocator must see no request at all during its calls.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from helpers import assert_bitexact

pytestmark = pytest.mark.gpu

WORKSPACE_BYTES = 8 << 20
WORKSPACE_EXCEEDED = 3


def say(text):
    print(text, flush=True)
    sys.stdout.flush()


def stats(hip):
    s = hip.MemoryStats()
    hip.call("spar_hip_memory_stats", ctypes.byref(s), 0)
    return (s.device_allocations, s.cache_hits, s.bytes_in_use)


def normal(hip, n, seed, dtype):
    buf = hip.DeviceBuffer(n * np.dtype(dtype).itemsize)
    hip.call("spar_hip_random_normal", buf.ptr, n, hip.dtype_tag(dtype), seed, 0.0, 1.0, 0)
    return buf


def out_bytes(outputs, dtype, op, hip):
    return outputs * (8 if op == hip.ARGMAX else np.dtype(dtype).itemsize)


def run_both(hip, x, shape, strides, offset, mask, dtype, op):
    """Both entry points on one view; returns (allocating, no-alloc) outputs."""
    rank = len(shape)
    outputs = int(np.prod([e for a, e in enumerate(shape) if not (mask >> a) & 1]))
    nbytes = out_bytes(outputs, dtype, op, hip)
    out_dtype = np.int64 if op == hip.ARGMAX else dtype
    ref = hip.DeviceBuffer(nbytes)
    got = hip.DeviceBuffer(nbytes)
    hip.call("spar_hip_zero", got.ptr, nbytes, 0)
    args = (rank, hip.u64_array(shape), hip.u64_array(strides), offset, mask,
            hip.dtype_tag(dtype), op, 0)
    hip.call("spar_hip_launch_axis_reduction", ref.ptr, x.ptr, *args)
    hip.synchronize()
    before = stats(hip)
    hip.call("spar_hip_launch_axis_reduction_no_alloc", got.ptr, x.ptr, *args)
    hip.synchronize()
    after = stats(hip)
    assert after == before, f"allocator used by the no-alloc call: {before} -> {after}"
    return ref.to_numpy(out_dtype, (outputs,)), got.to_numpy(out_dtype, (outputs,))


OPS = ["SUM", "MEAN", "MAX", "ARGMAX"]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("op", OPS)
def test_no_alloc_matches_allocating_entry_point(hip, dtype, op):
    code = getattr(hip, op)
    # Two calls in a row on the shared workspace, the second on a smaller
    # input: [8192, 8192] over axis 0 (a column split whose partials fill the
    # workspace for float32 argmax), then [1024, 2048] over axis 0.
    for rows, cols, seed in ((8192, 8192, 31), (1024, 2048, 32)):
        say(f"no_alloc {op} {np.dtype(dtype).name} [{rows},{cols}] axis 0")
        x = normal(hip, rows * cols, seed, dtype)
        want, got = run_both(hip, x, [rows, cols], [cols, 1], 0, 1, dtype, code)
        assert_bitexact(got, want, f"{op} axis 0 [{rows},{cols}]")
        del x


@pytest.mark.parametrize("op", OPS)
def test_no_alloc_layouts(hip, op):
    code = getattr(hip, op)
    dtype = np.float32
    x = normal(hip, 4096 * 8192, 33, dtype)
    cases = [
        # (label, shape, strides, offset, mask)
        ("rows axis 1", [4096, 8192], [8192, 1], 0, 2),
        ("full 2^25", [4096 * 8192], [1], 0, 1),
        ("few long rows", [4, 4096 * 2048], [4096 * 2048, 1], 0, 2),
        ("transposed view axis 1", [8192, 4096], [1, 8192], 0, 2),
        ("offset block axis 0", [3000, 5000], [8192, 1], 8192 * 7 + 64, 1),
        ("generic two axes", [64, 64, 2048], [64 * 8192, 8192, 1], 0, 5),
    ]
    for label, shape, strides, offset, mask in cases:
        last = offset + sum((e - 1) * s for e, s in zip(shape, strides))
        assert last < 4096 * 8192, label  # the view stays inside x
        say(f"no_alloc {op} {label}")
        want, got = run_both(hip, x, shape, strides, offset, mask, dtype, code)
        assert_bitexact(got, want, f"{op} {label}")
    # a second round on a smaller input reuses the workspace
    y = normal(hip, 257 * 1000, 34, dtype)
    say(f"no_alloc {op} [257,1000] axis 0 after the larger calls")
    want, got = run_both(hip, y, [257, 1000], [1000, 1], 0, 1, dtype, code)
    assert_bitexact(got, want, f"{op} [257,1000] axis 0")


def test_no_alloc_refuses_plans_beyond_the_workspace(hip):
    # float32 argmax over axis 0 of [32, (cus - 1) * 4096]: cus - 1 column
    # blocks of 4096 columns, one short of one block per CU, so the planner
    # splits the 32 rows in two, and the partials take 2 * cols values and
    # 2 * cols 32-bit indices (values rounded up to 256 bytes).  With more
    # than 128 CUs that exceeds the workspace, and the call must return
    # SPAR_HIP_STATUS_WORKSPACE_EXCEEDED and enqueue nothing.
    cus = hip.multiprocessor_count(0)
    cols = (cus - 1) * 4096
    rows = 32
    partial_bytes = -(-2 * cols * 4 // 256) * 256 + 2 * cols * 4
    if partial_bytes <= WORKSPACE_BYTES:
        pytest.skip(f"{cus} CUs: a [32, {cols}] argmax's partials fit the workspace")
    # MI355X: 256 CUs, 16,711,680 bytes of partials against 8 MiB
    x = normal(hip, rows * cols, 35, np.float32)
    out = hip.DeviceBuffer(cols * 8)
    sentinel = np.full(cols, -7, np.int64)
    hip.call("spar_hip_copy_host_to_device", out.ptr, sentinel.ctypes.data, sentinel.nbytes, 0)
    say(f"no_alloc ARGMAX [32, {cols}] axis 0 (expected refusal)")
    status = hip.status_of("spar_hip_launch_axis_reduction_no_alloc", out.ptr, x.ptr, 2,
                           hip.u64_array([rows, cols]), hip.u64_array([cols, 1]), 0, 1,
                           hip.FLOAT32, hip.ARGMAX, 0)
    hip.synchronize()
    assert status.code == WORKSPACE_EXCEEDED, (status.code, status.hip_error)
    assert np.array_equal(out.to_numpy(np.int64, (cols,)), sentinel)
    # the allocating entry point handles the same request
    hip.call("spar_hip_launch_axis_reduction", out.ptr, x.ptr, 2, hip.u64_array([rows, cols]),
             hip.u64_array([cols, 1]), 0, 1, hip.FLOAT32, hip.ARGMAX, 0)
    idx = out.to_numpy(np.int64, (cols,))
    host = x.to_numpy(np.float32, (rows, cols))
    assert np.array_equal(idx, np.argmax(host, axis=0))
