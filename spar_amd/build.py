"""Build recipe for the gfx950 backend and its host layers.

Produces, in-tree:
  spar_amd/lib/libspar_hip.so   HIP translation units (kernels + C ABI), hipcc
  spar_amd/lib/libspar.so       C++ host library (Tensor, ops, autograd), g++
  spar_amd/_spar*.so            pybind11 binding of the host library

Run `python -m spar_amd.build` (or call `build()`); every call recompiles.
"""
from __future__ import annotations

import concurrent.futures as futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
INCLUDE = ROOT / "include"
HIP_DIR = PACKAGE / "csrc" / "hip"
HOST_DIR = PACKAGE / "csrc" / "host"
PY_DIR = PACKAGE / "csrc" / "python"
MODULE_DIR = PACKAGE / "csrc" / "module"
LIB_DIR = PACKAGE / "lib"
OBJ_DIR = ROOT / "_build" / "spar_amd"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

# -ffp-contract=off keeps every multiply and add separately rounded, as on the
# CPU; the packed-fp32 feature is disabled so no v_pk_*_f32 is generated.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{HIP_DIR}",
]

HOST_FLAGS = [
    "-O2",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wextra",
    f"-I{INCLUDE}",
    f"-I{HOST_DIR / 'include'}",
]


def _run(command: list[str]) -> None:
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        sys.stderr.write(" ".join(command) + "\n" + result.stdout + result.stderr)
        raise RuntimeError(f"build step failed: {command[0]} ... {command[-1]}")


def _compile_hip(source: Path) -> Path:
    obj = OBJ_DIR / (source.stem + ".hip.o")
    _run([HIPCC, *HIP_FLAGS, "-c", str(source), "-o", str(obj)])
    return obj


def _compile_host(source: Path, extra: list[str] | None = None) -> Path:
    obj = OBJ_DIR / (source.stem + ".host.o")
    _run([CXX, *HOST_FLAGS, *(extra or []), "-c", str(source), "-o", str(obj)])
    return obj


def build_hip_library(jobs: int = 8) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(HIP_DIR.glob("*.hip"))
    with futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile_hip, sources))
    target = LIB_DIR / "libspar_hip.so"
    tmp = target.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, target)
    return target


def build_host_library(jobs: int = 8) -> Path:
    sources = sorted((HOST_DIR / "src").glob("*.cpp"))
    if not sources:
        raise RuntimeError("no host sources")
    with futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile_host, sources))
    target = LIB_DIR / "libspar.so"
    tmp = target.with_suffix(".so.tmp")
    _run([CXX, "-shared", "-fPIC", *map(str, objects), f"-L{LIB_DIR}", "-lspar_hip",
          "-Wl,-rpath,$ORIGIN", "-o", str(tmp)])
    os.replace(tmp, target)
    return target


def build_python_binding() -> Path:
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    target = PACKAGE / f"_spar{suffix}"
    tmp = PACKAGE / f"_spar{suffix}.tmp"
    source = PY_DIR / "bindings.cpp"
    _run([CXX, *HOST_FLAGS, "-shared", f"-I{pybind11.get_include()}",
          f"-I{sysconfig.get_paths()['include']}", "-fvisibility=hidden", str(source),
          f"-L{LIB_DIR}", "-lspar", "-lspar_hip", "-Wl,-rpath,$ORIGIN/lib", "-o", str(tmp)])
    os.replace(tmp, target)
    return target


def build_module_binding() -> Path:
    """Compiles spar.hip_ops (the C ABI as a C++23 named module, with
    spar_hip.h in its global module fragment) and a consumer that imports
    it, linked against libspar_hip.so: the binding Spar's own modules would
    use.  Returns the consumer executable."""
    clang = os.environ.get("CLANGXX", "/opt/rocm/llvm/bin/clang++")
    flags = ["-std=c++23", "-O2", f"-I{INCLUDE}"]
    pcm = OBJ_DIR / "spar_hip_ops.pcm"
    _run([clang, *flags, "--precompile", str(MODULE_DIR / "spar_hip_ops.cppm"), "-o", str(pcm)])
    module_obj = OBJ_DIR / "spar_hip_ops.o"
    _run([clang, "-std=c++23", "-O2", "-c", str(pcm), "-o", str(module_obj)])
    check_obj = OBJ_DIR / "module_check.o"
    _run([clang, *flags, f"-fmodule-file=spar.hip_ops={pcm}", "-c",
          str(MODULE_DIR / "module_check.cpp"), "-o", str(check_obj)])
    target = LIB_DIR / "spar_hip_module_check"
    _run([clang, str(check_obj), str(module_obj), f"-L{LIB_DIR}", "-lspar_hip",
          "-Wl,-rpath,$ORIGIN", "-o", str(target)])
    return target


def build(jobs: int = 8) -> None:
    build_hip_library(jobs)
    if (HOST_DIR / "src").exists() and any((HOST_DIR / "src").glob("*.cpp")):
        build_host_library(jobs)
        if (PY_DIR / "bindings.cpp").exists():
            build_python_binding()
    if MODULE_DIR.exists():
        build_module_binding()


def clean() -> None:
    shutil.rmtree(OBJ_DIR, ignore_errors=True)


if __name__ == "__main__":
    build()
