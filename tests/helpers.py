"""Shared numeric checks for the parity tests.

Tolerance classes (stated once, used everywhere):
  * bit-exact: identical bits for every non-NaN result; NaN positions equal
    (NaN payloads are not compared: the CPU and the GPU may quiet NaNs
    differently, and no op here defines a payload).
  * ulp(k): |a - b| <= k units in the last place of the float32 (or float64)
    reference, measured on the integer line of the format; infinities and
    NaNs must match exactly.
  * red(N): |gpu - cpu| <= 1e-6 * sqrt(N) * max(|cpu|, ||x||_2) for an
    N-element sum (the summation order differs; the scale is the natural
    magnitude of the sum, so a sum that cancels to ~0 is not judged
    relatively).
"""
from __future__ import annotations

import math

import numpy as np


def bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def assert_bitexact(got: np.ndarray, want: np.ndarray, what: str = "") -> None:
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert got.dtype == want.dtype, f"{what}: dtype {got.dtype} != {want.dtype}"
    if got.dtype.kind != "f":
        mismatch = np.flatnonzero(got.ravel() != want.ravel())
        assert mismatch.size == 0, f"{what}: {mismatch.size} mismatches, first at {mismatch[:5]}"
        return
    gn = np.isnan(got)
    wn = np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    g = bits(np.where(gn, 0, got).astype(got.dtype))
    w = bits(np.where(wn, 0, want).astype(want.dtype))
    mismatch = np.flatnonzero(g.ravel() != w.ravel())
    if mismatch.size:
        i = mismatch[0]
        raise AssertionError(
            f"{what}: {mismatch.size} of {got.size} differ; first at {i}: "
            f"got {got.ravel()[i]!r} want {want.ravel()[i]!r}")


def ordered_int(a: np.ndarray) -> np.ndarray:
    """Maps floats to integers that are monotonic in value (ulp distance)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.float32:
        i = a.view(np.int32).astype(np.int64)
        return np.where(i < 0, np.int64(-2**31) - i, i)
    i = a.view(np.int64)
    return np.where(i < 0, np.iinfo(np.int64).min - i, i)


def ulp_distance(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """Distance on the ordered-integer line, in int64 (exact; a difference
    that overflows int64 is reported as the int64 maximum)."""
    g = ordered_int(np.asarray(got))
    w = ordered_int(np.asarray(want))
    with np.errstate(over="ignore"):
        d = np.where(g >= w, g - w, w - g)
    return np.where(d < 0, np.iinfo(np.int64).max, d)


def assert_ulp(got: np.ndarray, want: np.ndarray, max_ulp: int, what: str = "") -> int:
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape and got.dtype == want.dtype, what
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    gi, wi = np.isinf(got), np.isinf(want)
    assert np.array_equal(gi, wi), f"{what}: inf positions differ"
    assert np.array_equal(got[gi], want[wi]), f"{what}: inf signs differ"
    finite = ~(gn | gi)
    if not finite.any():
        return 0
    d = ulp_distance(got[finite], want[finite])
    worst = int(d.max())
    if worst > max_ulp:
        i = int(np.argmax(d))
        raise AssertionError(
            f"{what}: max {worst} ulp > {max_ulp}; got {got[finite][i]!r} want {want[finite][i]!r}")
    return worst


def red_bound(n: int, reference, norm) -> float:
    return 1e-6 * math.sqrt(max(n, 1)) * np.maximum(np.abs(reference), norm)


def assert_red(got, want, n: int, norm, what: str = "") -> None:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    bound = red_bound(n, want, np.asarray(norm, dtype=np.float64))
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    with np.errstate(invalid="ignore"):  # inf - inf where both are the same infinity
        ok = gn | (np.abs(got - want) <= bound) | (got == want)
    if not ok.all():
        i = np.flatnonzero(~ok.ravel())[0]
        raise AssertionError(
            f"{what}: {int((~ok).sum())} outside red({n}); first {i}: got {got.ravel()[i]!r} "
            f"want {want.ravel()[i]!r} bound {np.broadcast_to(bound, got.shape).ravel()[i]!r}")


def special_values(dtype) -> np.ndarray:
    """IEEE edge values: signed zeros, denormals, extremes, infinities, NaN."""
    info = np.finfo(dtype)
    values = [0.0, -0.0, 1.0, -1.0, info.tiny, -info.tiny, info.tiny / 4, -info.tiny / 8,
              info.max, -info.max, info.eps, np.inf, -np.inf, np.nan, 0.5, 2.0, 3.0, 1e-3,
              -7.25, 88.0, -88.0, 100.0, -103.0, 1e30, -1e30]
    return np.array(values, dtype=dtype)
