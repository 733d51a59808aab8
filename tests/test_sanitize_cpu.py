"""The host library's sources and the oracle's C loops built with
AddressSanitizer and UndefinedBehaviorSanitizer (tests/sanitize/Makefile),
running host_checks.cpp on the CPU: shapes, views and their bounds, host
gathers, broadcast rules, view-only autograd graphs, the optimizer's host
logic, clean failures of device paths without a device, and the oracle's
strided loops.  The sanitizers abort on their first report."""
import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent / "sanitize"


def test_host_library_under_address_and_undefined_behaviour_sanitizers():
    build = subprocess.run(["make", "-s", "-j8", "-C", str(HERE)], capture_output=True, text=True,
                           timeout=600)
    assert build.returncode == 0, build.stdout[-3000:] + build.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    run = subprocess.run([str(HERE / "_build" / "host_checks")], capture_output=True, text=True,
                         timeout=300, env=env)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-3000:]
    assert "host checks: 0 failure(s)" in run.stdout
