"""The oracle's C under sanitizers (CPU only).

oracle/sanitize_check.c drives every oracle entry point on small edge-case
inputs (NaN, +-inf, ragged sizes, threaded forms) and checks properties the
mathematics fixes; `make -C oracle sanitize` builds it with
AddressSanitizer + UndefinedBehaviorSanitizer and with ThreadSanitizer and
runs both.  A report from either sanitizer, or a failed check, fails the run.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None and shutil.which("cc") is None,
                    reason="no C compiler")
def test_oracle_under_asan_ubsan_and_tsan():
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:abort_on_error=0"
    env["TSAN_OPTIONS"] = "halt_on_error=1"
    r = subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle"), "sanitize"],
                       capture_output=True, text=True, env=env, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert out.count("sanitize_check: all checks passed") == 2, out[-4000:]
