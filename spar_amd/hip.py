"""ctypes binding of the backend's C ABI (include/spar_hip.h).

This is the FFI stub a Python caller uses to reach the kernels directly with
raw device pointers; the C++ host library (spar_amd._spar) reaches the same
entry points from C++.  Loading fails loudly if the library is not built:
there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "lib" / "libspar_hip.so"

FLOAT32, FLOAT64, INT32, INT64 = 0, 1, 2, 3
ADD, SUBTRACT, MULTIPLY, DIVIDE = 0, 1, 2, 3
EQUAL, NOT_EQUAL, LESS, LESS_EQUAL, GREATER, GREATER_EQUAL = 4, 5, 6, 7, 8, 9
NEGATE, SQUARE, RECIPROCAL, EXP, LOG, SQRT, SIGMOID, SILU, TANH, GELU, GELU_DERIVATIVE = range(11)
SUM, MEAN, MAX, ARGMAX = 0, 1, 2, 3
MAX_RANK = 8

BINARY_OPS = {"add": ADD, "subtract": SUBTRACT, "multiply": MULTIPLY, "divide": DIVIDE,
              "equal": EQUAL, "not_equal": NOT_EQUAL, "less": LESS, "less_equal": LESS_EQUAL,
              "greater": GREATER, "greater_equal": GREATER_EQUAL}
UNARY_OPS = {"negate": NEGATE, "square": SQUARE, "reciprocal": RECIPROCAL, "exp": EXP,
             "log": LOG, "sqrt": SQRT, "sigmoid": SIGMOID, "silu": SILU, "tanh": TANH,
             "gelu": GELU, "gelu_derivative": GELU_DERIVATIVE}

_DTYPE_TAGS = {np.dtype(np.float32): FLOAT32, np.dtype(np.float64): FLOAT64,
               np.dtype(np.int32): INT32, np.dtype(np.int64): INT64}


class Status(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int), ("hip_error", ctypes.c_int)]


class MemoryStats(ctypes.Structure):
    _fields_ = [("bytes_in_use", ctypes.c_uint64), ("bytes_cached", ctypes.c_uint64),
                ("bytes_reserved", ctypes.c_uint64), ("device_allocations", ctypes.c_uint64),
                ("cache_hits", ctypes.c_uint64)]


class NormSummary(ctypes.Structure):
    _fields_ = [("scale", ctypes.c_double), ("scaled_sum_squares", ctypes.c_double),
                ("has_infinity", ctypes.c_int), ("has_nan", ctypes.c_int)]


class HipError(RuntimeError):
    def __init__(self, name: str, status: Status, message: str):
        super().__init__(f"{name} failed: {message} (code {status.code}, hip error {status.hip_error})")
        self.code = status.code
        self.hip_error = status.hip_error


_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_U32 = ctypes.c_uint32
_I = ctypes.c_int
_D = ctypes.c_double
_U64P = ctypes.POINTER(ctypes.c_uint64)

# name -> argument types (every entry point returns Status except error_string and
# norm_max_extent)
SIGNATURES = {
    "spar_hip_device_count": [ctypes.POINTER(ctypes.c_int)],
    "spar_hip_multiprocessor_count": [ctypes.POINTER(ctypes.c_int), _I],
    "spar_hip_allocate": [ctypes.POINTER(ctypes.c_void_p), _U64, _I],
    "spar_hip_deallocate": [_P, _I],
    "spar_hip_empty_cache": [_I],
    "spar_hip_memory_stats": [ctypes.POINTER(MemoryStats), _I],
    "spar_hip_zero": [_P, _U64, _I],
    "spar_hip_touch": [_P, _U64, _P, _I],
    "spar_hip_copy_host_to_device": [_P, _P, _U64, _I],
    "spar_hip_copy_device_to_host": [_P, _P, _U64, _I],
    "spar_hip_copy_device_to_device": [_P, _I, _P, _I, _U64],
    "spar_hip_synchronize": [_I],
    "spar_hip_stream": [ctypes.POINTER(ctypes.c_void_p), _I],
    "spar_hip_event_create": [ctypes.POINTER(ctypes.c_void_p)],
    "spar_hip_event_destroy": [_P],
    "spar_hip_event_record": [_P, _I],
    "spar_hip_event_elapsed": [ctypes.POINTER(ctypes.c_float), _P, _P],
    "spar_hip_launch_binary": [_P, _P, _P, _U64, _I, _I, _I],
    "spar_hip_launch_scalar": [_P, _P, _U64, _I, _I, _D, _I],
    "spar_hip_launch_unary": [_P, _P, _U64, _I, _I, _I],
    "spar_hip_launch_fill_from_scalar": [_P, _P, _U64, _I, _D, _I],
    "spar_hip_launch_fill_from_scalar_divided": [_P, _P, _U64, _I, _D, _I],
    "spar_hip_launch_fill": [_P, _U64, _I, _D, _I],
    "spar_hip_launch_add_in_place": [_P, _P, _U64, _I, _I],
    "spar_hip_launch_strided_copy": [_P, _P, _U64, _U64P, _U64P, _U64, _U64, _U64, _I],
    "spar_hip_launch_strided_assign": [_P, _U64, _U64P, _U64P, _U64, _P, _U64, _I],
    "spar_hip_launch_strided_binary": [_P, _P, _U64P, _U64, _P, _U64P, _U64, _U64, _U64P, _I, _I,
                                       _I],
    "spar_hip_launch_reduction": [_P, _P, _U64, _I, _I, _I],
    "spar_hip_launch_row_reduction": [_P, _P, _U64, _U64, _I, _I, _I],
    "spar_hip_launch_axis_reduction": [_P, _P, _U64, _U64P, _U64P, _U64, _U32, _I, _I, _I],
    "spar_hip_launch_axis_reduction_no_alloc": [_P, _P, _U64, _U64P, _U64P, _U64, _U32, _I, _I,
                                                _I],
    "spar_hip_launch_broadcast_reduce": [_P, _P, _U64, _U64P, _U64, _U64P, _U64P, _U64, _I, _I],
    "spar_hip_launch_multiply_reduce": [_P, _P, _P, _U64, _U64P, _U64, _U64P, _U64, _I, _I],
    "spar_hip_launch_probability_forward": [_P, _P, _P, _U64, _U64, _U64, _I, _I, _I],
    "spar_hip_launch_probability_backward": [_P, _P, _P, _P, _U64, _U64, _U64, _I, _I, _I],
    "spar_hip_launch_window_embed": [_P, _P, _U64, _U64, _U64, _U64, _U64, _U64, _I],
    "spar_hip_launch_box_embed": [_P, _P, _I, _P, _P, _P, _U64, _I],
    "spar_hip_launch_norm_forward": [_P, _P, _P, _P, _U64, _U64, _P, _P, _U64, _U64, _D, _I, _I,
                                     _I],
    "spar_hip_launch_norm_backward": [_P, _U64, _P, _P, _P, _P, _U64, _U64, _P, _P, _P, _U64,
                                      _U64, _I, _I, _I],
    "spar_hip_launch_norm_backward_scaled": [_P, _U64, _P, _P, _P, _P, _P, _U64, _U64, _P, _P,
                                             _P, _U64, _U64, _I, _I, _I],
    "spar_hip_validate_targets": [ctypes.POINTER(ctypes.c_int32), _P, _U64, _U64, _I, _I],
    "spar_hip_launch_nll_forward": [_P, _P, _P, _U64, _U64, _U64, _I, _I, _I, _I],
    "spar_hip_launch_nll_backward": [_P, _P, _P, _U64, _U64, _U64, _I, _I, _I, _I],
    "spar_hip_launch_cross_entropy_forward": [_P, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _I, _I,
                                              _I, _I],
    "spar_hip_launch_cross_entropy_backward": [_P, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _I,
                                               _I, _I, _I],
    "spar_hip_gradient_norm_summary": [ctypes.POINTER(NormSummary), _P, _U64, _I, _I],
    "spar_hip_launch_gradient_norm_summary": [_P, _P, _U64, _I, _I],
    "spar_hip_launch_scale_in_place": [_P, _U64, _I, _D, _I],
    "spar_hip_launch_adamw": [_P, _P, _P, _P, _U64, _I, _D, _D, _D, _D, _D, _D, _D, _I],
    "spar_hip_random_uniform": [_P, _U64, _I, _U64, _D, _D, _I],
    "spar_hip_random_normal": [_P, _U64, _I, _U64, _D, _D, _I],
}

_lib = None


def library_path() -> Path:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Loads libspar_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise ImportError(f"{_LIB_PATH} is not built; run `python -m spar_amd.build`")
    lib = ctypes.CDLL(str(_LIB_PATH), mode=os.RTLD_NOW | ctypes.RTLD_GLOBAL)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = Status
    lib.spar_hip_error_string.argtypes = [ctypes.c_int]
    lib.spar_hip_error_string.restype = ctypes.c_char_p
    lib.spar_hip_norm_max_extent.argtypes = [ctypes.c_int]
    lib.spar_hip_norm_max_extent.restype = ctypes.c_uint64
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Calls a C-ABI entry point and raises HipError on a non-zero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status.code != 0:
        message = lib.spar_hip_error_string(status.hip_error)
        raise HipError(name, status, message.decode() if message else "unknown error")


def status_of(name: str, *args) -> Status:
    """Calls an entry point and returns its status without raising."""
    return getattr(load(), name)(*args)


def u64_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (ctypes.c_uint64 * max(len(values), 1))(*values)


def dtype_tag(dtype) -> int:
    return _DTYPE_TAGS[np.dtype(dtype)]


def multiprocessor_count(device: int = 0) -> int:
    count = ctypes.c_int(0)
    call("spar_hip_multiprocessor_count", ctypes.byref(count), device)
    return count.value


def device_count() -> int:
    count = ctypes.c_int(0)
    call("spar_hip_device_count", ctypes.byref(count))
    return count.value


def synchronize(device: int = 0) -> None:
    call("spar_hip_synchronize", device)


class DeviceBuffer:
    """Device memory from the backend's caching allocator."""

    def __init__(self, nbytes: int, device: int = 0):
        self.nbytes = int(nbytes)
        self.device = device
        pointer = ctypes.c_void_p()
        call("spar_hip_allocate", ctypes.byref(pointer), self.nbytes, device)
        self.ptr = pointer.value or 0

    @classmethod
    def from_numpy(cls, array: np.ndarray, device: int = 0) -> "DeviceBuffer":
        array = np.ascontiguousarray(array)
        buffer = cls(array.nbytes, device)
        if array.nbytes:
            call("spar_hip_copy_host_to_device", buffer.ptr, array.ctypes.data, array.nbytes, device)
        return buffer

    def to_numpy(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("requested view exceeds the buffer")
        if out.nbytes:
            call("spar_hip_copy_device_to_host", out.ctypes.data, self.ptr, out.nbytes, self.device)
        return out

    def address(self, byte_offset: int = 0) -> int:
        return self.ptr + byte_offset

    def free(self) -> None:
        if self.ptr:
            call("spar_hip_deallocate", self.ptr, self.device)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        handle = ctypes.c_void_p()
        call("spar_hip_event_create", ctypes.byref(handle))
        self.handle = handle.value

    def record(self, device: int = 0) -> None:
        call("spar_hip_event_record", self.handle, device)

    def elapsed_ms(self, stop: "Event") -> float:
        ms = ctypes.c_float()
        call("spar_hip_event_elapsed", ctypes.byref(ms), self.handle, stop.handle)
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                call("spar_hip_event_destroy", self.handle)
        except Exception:
            pass
