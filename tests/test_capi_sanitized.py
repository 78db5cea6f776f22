"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer: the library
is rebuilt with host-side instrumentation (tests/sanitize/build_asan.py) and its argument
checking driven through every refusal path (tests/sanitize/drive_capi.py) in a subprocess
with the clang ASan runtime preloaded.  CPU only: every call is refused before a launch."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_capi_host_checks_are_clean_under_asan_and_ubsan(tmp_path):
    sys.path.insert(0, os.path.join(HERE, "sanitize"))
    try:
        import build_asan
    finally:
        sys.path.pop(0)
    lib = build_asan.build(str(tmp_path))
    syms = subprocess.run(["nm", "-D", "--undefined-only", lib], capture_output=True, text=True,
                          check=True).stdout
    assert "__asan_init" in syms and "__ubsan_handle" in syms, "host code not instrumented"
    env = dict(os.environ, LD_PRELOAD=build_asan.asan_runtime(),
               ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    proc = subprocess.run([sys.executable, os.path.join(HERE, "sanitize", "drive_capi.py"), lib],
                          capture_output=True, text=True, env=env, timeout=300)
    report = proc.stdout + proc.stderr
    assert proc.returncode == 0, report[-4000:]
    assert "AddressSanitizer" not in report and "runtime error" not in report, report[-4000:]
    assert proc.stdout.startswith("OK ") and int(proc.stdout.split()[1]) >= 30
