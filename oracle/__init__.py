"""The oracle: a CPU restatement of Spar's CPU path (TEST INFRASTRUCTURE ONLY).

`oracle/spar_oracle.c` restates the reference's CPU loops in C (compiled by
`oracle/Makefile` with -O2 -ffp-contract=off); this module binds it with
ctypes and adds numpy helpers.  `oracle.reference` restates the host-side
tensor logic (views, broadcast, autograd) in Python on top of these loops.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import
this package, always as the reference results are compared with; the
product (spar_amd/) never does.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libspar_oracle.so"

_lib = None

_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_U32 = ctypes.c_uint32
_I = ctypes.c_int
_I64 = ctypes.c_int64
_D = ctypes.c_double
_U64P = ctypes.POINTER(ctypes.c_uint64)


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _typed(name, restype, argtypes):
    return name, restype, argtypes


def _signatures():
    sigs = [
        ("spar_oracle_next_u64", _U64, [_U64P]),
        ("spar_oracle_uniform_float", ctypes.c_float, [_U64P]),
        ("spar_oracle_uniform_double", _D, [_U64P]),
        ("spar_oracle_strided_copy", None, [_P, _P, _U64, _U64, _U64P, _U64P, _U64]),
        ("spar_oracle_adamw_correction", _D, [_D, _U64]),
    ]
    for suffix, scalar in (("f32", ctypes.c_float), ("f64", ctypes.c_double)):
        sigs += [
            (f"spar_oracle_random_uniform_{suffix}", None, [_P, _U64, _U64P, _D, _D]),
            (f"spar_oracle_random_normal_{suffix}", None, [_P, _U64, _U64P, _D, _D]),
            (f"spar_oracle_binary_{suffix}", None, [_P, _P, _U64P, _U64, _P, _U64P, _U64, _U64, _U64P, _I]),
            (f"spar_oracle_scalar_{suffix}", None, [_P, _P, _U64, _I, _D]),
            (f"spar_oracle_unary_{suffix}", None, [_P, _P, _U64, _I]),
            (f"spar_oracle_sum_{suffix}", scalar, [_P, _U64, _U64P, _U64P, _U64]),
            (f"spar_oracle_mean_{suffix}", scalar, [_P, _U64, _U64P, _U64P, _U64]),
            (f"spar_oracle_max_{suffix}", scalar, [_P, _U64, _U64P, _U64P, _U64]),
            (f"spar_oracle_axis_sum_{suffix}", None, [_P, _U64, _P, _U64, _U64P, _U64P, _U64, _U32]),
            (f"spar_oracle_axis_max_{suffix}", None, [_P, _P, _U64, _P, _U64, _U64P, _U64P, _U64, _U32, _P]),
            (f"spar_oracle_reduce_gradient_{suffix}", None, [_P, _P, _U64, _U64P, _U64P, _U64, _U64, _U64P]),
            (f"spar_oracle_add_in_place_{suffix}", None, [_P, _P, _U64]),
            (f"spar_oracle_fill_{suffix}", None, [_P, _U64, scalar]),
            (f"spar_oracle_softmax_axis_{suffix}", None, [_P, _P, _P, _U64, _U64P, _U64P, _U64, _U64]),
            (f"spar_oracle_softmax_full_{suffix}", None, [_P, _P, _U64]),
            (f"spar_oracle_softmax_full_undefined_{suffix}", _I, [_P, _U64]),
            (f"spar_oracle_softmax_axis_backward_{suffix}", None, [_P, _P, _P, _P, _U64, _U64P, _U64]),
            (f"spar_oracle_softmax_full_backward_{suffix}", None, [_P, _P, _P, _U64, _I]),
            (f"spar_oracle_log_softmax_{suffix}", None, [_P, _P, _P, _U64, _U64P, _U64P, _U64, _I64]),
            (f"spar_oracle_log_softmax_backward_{suffix}", None, [_P, _P, _P, _P, _U64, _U64, _U64]),
            (f"spar_oracle_adamw_{suffix}", None, [_P, _P, _P, _P, _U64, _D, _D, _D, _D, _D, _D, _D]),
            (f"spar_oracle_sum_squares_add_{suffix}", None, [_P, _P, _P, _U64]),
            (f"spar_oracle_scale_{suffix}", None, [_P, _U64, _D]),
        ]
    return sigs


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, restype, argtypes in _signatures():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def u64(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (ctypes.c_uint64 * max(len(values), 1))(*values)


def suffix_of(dtype) -> str:
    dtype = np.dtype(dtype)
    if dtype == np.float32:
        return "f32"
    if dtype == np.float64:
        return "f64"
    raise TypeError(f"oracle supports float32/float64, not {dtype}")


def ptr(array: np.ndarray) -> int:
    return array.ctypes.data


def fn(name: str, dtype):
    return getattr(lib(), f"{name}_{suffix_of(dtype)}")
