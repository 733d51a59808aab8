"""Recipe for compiling the reference's own CPU path into oracle/_ref/ (checker only).

The reference is C++23 named modules whose every unit starts with
`import std;` (its CMakeLists.txt requires CMake's import-std support and
C++ module scanning).  This image has clang 22 with libstdc++ 11: no
standard-library module (`std.cppm`), no libc++ headers and no
clang-scan-deps, so no reference translation unit compiles here without
rewriting its sources, which this recipe does not do.  `build()` probes the
toolchain for `import std` and, while that probe fails, records the reason
in oracle/_ref/UNBUILDABLE and builds nothing; the oracle is then pinned by
the checks described in the tests (closed forms, library routines, brute
force) instead of a reference binary.
"""
from __future__ import annotations

import os
import subprocess
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
REF_OUT = HERE / "_ref"
REFERENCE = Path("/root/reference")


def probe_import_std(compiler: str = "/opt/rocm/llvm/bin/clang++") -> tuple[bool, str]:
    with tempfile.TemporaryDirectory() as tmp:
        source = Path(tmp) / "probe.cpp"
        source.write_text("import std;\nint main() { std::vector<int> v{1}; return v[0] - 1; }\n")
        result = subprocess.run([compiler, "-std=c++23", "-c", str(source), "-o",
                                 str(Path(tmp) / "probe.o")], capture_output=True, text=True)
        return result.returncode == 0, (result.stderr or result.stdout).strip().splitlines()[:3]


def build() -> bool:
    """Returns True if a reference build was produced (never, on this image)."""
    if not REFERENCE.exists():
        return False
    REF_OUT.mkdir(exist_ok=True)
    ok, detail = probe_import_std()
    if not ok:
        (REF_OUT / "UNBUILDABLE").write_text(
            "The reference's translation units use `import std;` (C++23 standard library "
            "modules); this toolchain cannot compile it:\n" + "\n".join(detail) + "\n")
        return False
    # A toolchain with `import std` would build the reference's CPU sources
    # from /root/reference here; none is available in this image.
    (REF_OUT / "UNBUILDABLE").write_text("import std compiles, but no recipe is written for it\n")
    return False


if __name__ == "__main__":
    print("reference built:", build())
    marker = REF_OUT / "UNBUILDABLE"
    if marker.exists():
        print(marker.read_text())
