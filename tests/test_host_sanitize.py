"""libtkv_hip's host code under AddressSanitizer + UndefinedBehaviorSanitizer.

`make -C tokenvector/inference_amd/csrc sanitize` builds every library source
with the sanitizers on the host side only (device code is built as for the
shipped library) and links them with tests/native/host_sanitize.cpp, a C
program that drives the C ABI.  Without a GPU the program exercises the
argument checks and the no-device error paths; on a GPU it also runs small
calls of every entry point family, weights, the static entry, forced GEMM
configurations, graphs with workspace growth and both teardown orders of a
context and its graph.  A sanitizer report or a failed check exits non-zero.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tokenvector", "inference_amd", "csrc")
EXE = os.path.join(CSRC, "_build_san", "host_sanitize")


def _run(gpu: bool):
    env = dict(os.environ)
    # the ROCm runtime's own allocations outlive main(); leaks are not what
    # this run looks for
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0" + (":protect_shadow_gap=0" if gpu else "")
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    return subprocess.run([EXE], capture_output=True, text=True, env=env, timeout=300)


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="no hipcc")
def test_library_host_code_sanitized_without_device():
    r = subprocess.run(["make", "-s", "-j8", "-C", CSRC, "_build_san/host_sanitize"],
                       capture_output=True, text=True, timeout=1500)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    env_has_gpu = False
    try:
        import torch
        env_has_gpu = torch.cuda.device_count() > 0
    except Exception:
        pass
    if env_has_gpu:
        pytest.skip("a GPU is visible: the device run is the gpu-marked test")
    r = _run(gpu=False)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "host_sanitize: all checks passed (no device)" in out, out[-4000:]


@pytest.mark.gpu
def test_library_host_code_sanitized_on_device():
    assert os.path.exists(EXE), "sanitized build missing: run `make -C %s sanitize` first" % CSRC
    r = _run(gpu=True)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "host_sanitize: all checks passed (device 0)" in out, out[-4000:]
