"""C-ABI library checks that need no GPU: every symbol include/spar_hip.h
declares is exported, and invalid arguments are rejected on the host with
status code 1 before any device call (the reference's convention,
src/backend/cuda_kernels.cu:12-22, :714-720)."""
import ctypes
import re
from pathlib import Path

import pytest

from spar_amd import hip

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "spar_hip.h").read_text()
    return sorted(set(re.findall(r"\b(spar_hip_\w+)\s*\(", text)))


def test_header_symbols_exported():
    lib = ctypes.CDLL(str(hip.library_path()))
    names = declared_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # the Python binding describes every declared entry point
    assert set(names) - {"spar_hip_error_string", "spar_hip_norm_max_extent"} == set(hip.SIGNATURES)


def test_host_library_and_binding_load():
    lib = ctypes.CDLL(str(ROOT / "spar_amd" / "lib" / "libspar.so"))
    assert lib is not None
    from spar_amd import spar

    assert spar.hip_device_count() >= 0


U = hip.u64_array


@pytest.mark.parametrize("name,args", [
    ("spar_hip_launch_binary", (None, None, None, 4, 7, 0, 0)),        # bad dtype
    ("spar_hip_launch_binary", (None, None, None, 4, 0, 42, 0)),       # bad op
    ("spar_hip_launch_binary", (None, None, None, 4, 0, 0, 0)),        # null pointers
    ("spar_hip_launch_scalar", (None, None, 4, 0, 5, 1.0, 0)),         # compare op as scalar op
    ("spar_hip_launch_unary", (None, None, 4, 2, 0, 0)),               # int dtype
    ("spar_hip_launch_unary", (None, None, 4, 0, 11, 0)),              # bad op
    ("spar_hip_launch_reduction", (None, None, 4, 0, 0, 0)),           # null output
    ("spar_hip_launch_row_reduction", (None, None, 2, 0, 0, 1, 0)),    # mean of empty rows
    ("spar_hip_launch_strided_copy", (None, None, 1, U([4]), U([1]), 0, 4, 2, 0)),  # element size
    ("spar_hip_launch_strided_copy", (None, None, 9, U([1] * 9), U([1] * 9), 0, 1, 4, 0)),  # rank
    ("spar_hip_launch_axis_reduction", (None, None, 2, U([2, 2]), U([2, 1]), 0, 4, 0, 0, 0)),  # mask
    ("spar_hip_launch_broadcast_reduce", (None, None, 1, U([4]), 2, U([1, 4]), U([0, 0]), 4, 0, 0)),
    ("spar_hip_launch_probability_forward", (None, None, None, 1, 0, 1, 0, 0, 0)),  # empty axis
    ("spar_hip_launch_probability_forward", (None, None, None, 1, 4, 1, 0, 2, 0)),  # log flag
    ("spar_hip_launch_probability_backward", (None, None, None, None, 1, 4, 0, 0, 0, 0)),
    ("spar_hip_launch_fill_from_scalar", (None, None, 4, 0, 0.25, 0)),  # null scalar
    ("spar_hip_launch_fill_from_scalar_divided", (None, None, 4, 0, 0.0, 0)),  # divisor 0
    ("spar_hip_random_uniform", (None, 4, 0, 1, 1.0, 1.0, 0)),         # low == high
])
def test_invalid_arguments_rejected_on_host(name, args):
    status = hip.status_of(name, *args)
    assert status.code == 1, f"{name}{args} -> {status.code}"


@pytest.mark.parametrize("name,args", [
    ("spar_hip_launch_binary", (None, None, None, 0, 0, 0, 0)),
    ("spar_hip_launch_unary", (None, None, 0, 1, 3, 0)),
    ("spar_hip_launch_add_in_place", (None, None, 0, 0, 0)),
    ("spar_hip_launch_strided_copy", (None, None, 0, None, None, 0, 0, 4, 0)),
    ("spar_hip_zero", (None, 0, 0)),
    ("spar_hip_copy_host_to_device", (None, None, 0, 0)),
])
def test_zero_count_succeeds_without_device(name, args):
    assert hip.status_of(name, *args).code == 0


def test_error_string():
    lib = hip.load()
    assert lib.spar_hip_error_string(0)
    assert lib.spar_hip_error_string(1)


def test_module_binding_compiles_and_calls_the_abi():
    """spar.hip_ops (spar_amd/csrc/module/spar_hip_ops.cppm) is a C++23 named
    module with spar_hip.h in its global module fragment, as Spar's backend
    modules include the CUDA header (src/backend/cuda_ops.cppm:1-5); build()
    compiles it with clang++ --precompile and links a consumer that imports
    it.  The module wraps every in-scope function of the reference's
    spar.cuda_ops (cuda_ops.cppm:33-65: binary, scalar, unary, reduction,
    row_reduction, probability forward and backward, fill_from_device_scalar,
    validate_targets, nll forward and backward, gradient_norm_summary,
    scale_in_place, adamw_update); the consumer drives each through its
    host-only paths: empty launches succeed, invalid arguments become
    std::invalid_argument, the module's own checks std::logic_error."""
    import subprocess

    binary = ROOT / "spar_amd" / "lib" / "spar_hip_module_check"
    assert binary.exists(), "build() did not produce the module consumer"
    run = subprocess.run([str(binary)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "empty launch ok, invalid dtype rejected" in run.stdout
    assert ", 0 failed;" in run.stdout
    lines = [line for line in run.stdout.splitlines() if line.startswith(("ok", "FAIL"))]
    assert lines and all(line.startswith("ok") for line in lines), run.stdout
    wrappers = {line.split()[1].rstrip(",:") for line in lines}
    assert wrappers == {"binary", "scalar", "unary", "reduction", "row_reduction",
                        "probability_forward", "probability_backward",
                        "fill_from_device_scalar", "validate_targets", "nll_forward",
                        "nll_backward", "gradient_norm_summary", "scale_in_place",
                        "adamw_update"}, wrappers