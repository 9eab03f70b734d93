"""The C ABI's failure convention, checked where it can run without a GPU.

The reference's caller runs its own .tkv loop whenever a native entry point
returns rc < 0 (docs/HANDOFF.md:3649), and an environment flag gates the
native path.  Here: every host mirror returns TKV_HIP_NO_DEVICE (-2) in a
process that sees no gfx950 device (this container), TKV_HIP_UNSUPPORTED
(-1) when TKV_QUANT_HIP=0 (checked in a fresh process, since the gate is
read once), and TKV_HIP_BAD_ARG (-4) exactly where the .tkv function
raises ValueError, before any device is touched.
"""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

from tokenvector.inference_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _err():
    buf = C.create_string_buffer(512)
    _lib.lib().tkv_hip_last_error(buf, 512)
    return buf.value.decode()


@pytest.fixture(scope="module")
def nodev():
    L = _lib.lib()
    if L.tkv_hip_device_count() > 0:
        pytest.skip("a gfx950 device is visible: the no-device path cannot be observed")
    return L


def test_host_mirrors_return_no_device(nodev):
    L = nodev
    x = np.linspace(-1, 1, 64, dtype=np.float32)
    scale, mn, mx = C.c_float(), C.c_float(), C.c_float()
    zp = C.c_int64()
    rc = L.tkv_hip_calibrate_minmax(_p(x), x.size, 1, C.byref(scale), C.byref(zp), C.byref(mn),
                                    C.byref(mx))
    assert rc == _lib.NO_DEVICE and "device" in _err()
    q = np.zeros(64, np.int32)
    assert L.tkv_hip_quantize_int8_symmetric(_p(x), 64, _p(q), 64, C.c_float(0.01)) == _lib.NO_DEVICE
    a = np.ones(4 * 8, np.int32)
    y = np.zeros(4 * 4, np.float32)
    sw = np.ones(4, np.float32)
    rc = L.tkv_hip_matmul_int8_per_channel(_p(a), _p(a), None, 0, _p(y), 4, 4, 8, C.c_float(1.0),
                                           _p(sw), 4)
    assert rc == _lib.NO_DEVICE
    h = C.c_int64()
    assert L.tkv_hip_ctx_create(0, C.byref(h)) == _lib.NO_DEVICE
    # device entry points on the thread's default context fail the same way
    assert L.tkv_hip_dev_quantize_fp8_e4m3(0, None, 0, None) == _lib.NO_DEVICE


def test_bad_arguments_before_device(nodev):
    """ValueError cases of the .tkv functions are reported as BAD_ARG even
    without a device (the caller raises, it does not fall back)."""
    L = nodev
    a = np.ones(4 * 8, np.int32)
    y = np.zeros(4 * 4, np.float32)
    sw = np.ones(3, np.float32)                    # scales shorter than N (matmul.tkv:18-19)
    rc = L.tkv_hip_matmul_int8_per_channel(_p(a), _p(a), None, 0, _p(y), 4, 4, 8, C.c_float(1.0),
                                           _p(sw), 3)
    assert rc == _lib.BAD_ARG, rc
    x = np.ones(16, np.float32)
    q = np.zeros(8, np.int32)                      # dst shorter than src (engine.tkv:217-218)
    assert L.tkv_hip_quantize_int8_symmetric(_p(x), 16, _p(q), 8, C.c_float(0.1)) == _lib.BAD_ARG
    with pytest.raises(ValueError):
        _lib.check(_lib.BAD_ARG)


def test_env_gate_makes_mirrors_unsupported():
    """TKV_QUANT_HIP=0: every host mirror returns -1 so the .tkv caller keeps
    its own loop (whether or not a device is present)."""
    code = (
        "import ctypes as C, numpy as np\n"
        "from tokenvector.inference_amd import _lib\n"
        "L = _lib.lib()\n"
        "x = np.ones(64, np.float32); q = np.zeros(64, np.int32)\n"
        "p = lambda a: a.ctypes.data_as(C.c_void_p)\n"
        "s, mn, mx = C.c_float(), C.c_float(), C.c_float(); zp = C.c_int64()\n"
        "r1 = L.tkv_hip_calibrate_minmax(p(x), 64, 1, C.byref(s), C.byref(zp), C.byref(mn), C.byref(mx))\n"
        "r2 = L.tkv_hip_quantize_int8_symmetric(p(x), 64, p(q), 64, C.c_float(0.1))\n"
        "r3 = L.tkv_hip_quantize_fp8_e4m3(p(x), 64, p(q), 64)\n"
        "print(r1, r2, r3)\n"
    )
    env = dict(os.environ, TKV_QUANT_HIP="0", PYTHONPATH=ROOT)
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=120, cwd=ROOT)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == [str(_lib.UNSUPPORTED)] * 3, out.stdout
