"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

tests/c_abi/sanitize_check.c drives the no-device paths of the C ABI (storage, argument
errors, PQ training and encoding on the host, compared bit for bit with the oracle) through
a build whose host code -- the oracle, the host PQ trainer and the host pass of px_index.hip
-- is instrumented (tests/c_abi/Makefile, target `sanitize`). A memory error, a leak of this
project's code or undefined behaviour fails the run; the runtimes' own lifetime allocations
are suppressed by tests/c_abi/lsan.supp.
"""
import os
import subprocess

import pytest

from proxima_amd import _lib

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.mark.skipif(_lib.device_count() > 0, reason="checks the host paths without a device")
def test_host_code_under_sanitizers():
    build = subprocess.run(["make", "-s", "-C", os.path.join(HERE, "c_abi"), "sanitize"],
                           capture_output=True, text=True, timeout=900)
    assert build.returncode == 0, build.stderr[-4000:]
    env = dict(os.environ,
               ASAN_OPTIONS="detect_leaks=1",
               LSAN_OPTIONS="suppressions=" + os.path.join(HERE, "c_abi", "lsan.supp"),
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    run = subprocess.run([os.path.join(ROOT, "_build", "asan", "sanitize_check")], env=env,
                         capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, (run.stdout[-2000:], run.stderr[-6000:])
    assert "sanitize_check ok" in run.stdout
    assert "ERROR: AddressSanitizer" not in run.stderr and "runtime error" not in run.stderr
