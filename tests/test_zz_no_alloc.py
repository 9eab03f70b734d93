"""tkv_hip_linear_forward_static (fixed per-GPU scratch, no allocation)
against tkv_hip_linear_forward on the same weights and inputs, bit for bit:
two calls in a row per activation mode, the second with a smaller input,
covering every path the static entry reaches (per-tensor calibrate +
quantize + tiled GEMM, the single-pass calibrate + quantize of 64 MB and
larger activations across a reset of its barrier slots, the split-K skinny
GEMM at m <= 32, the one-kernel per-token decode linear, the per-token
rowwise quantize + GEMM); then a size beyond the scratch is refused.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle as O
from tokenvector.inference_amd import _lib
from tokenvector.inference_amd import device as D

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _static(lin, dx, m, mode, dy, stream):
    return _lib.lib().tkv_hip_linear_forward_static(lin.handle, C.c_void_p(dx.ptr), int(m),
                                                    int(mode), C.c_void_p(dy.ptr), stream)


@pytest.mark.parametrize("mode,ms", [(D.ACT_PER_TENSOR, (1024, 300)), (D.ACT_PER_TENSOR, (32, 4)),
                                     (D.ACT_PER_TOKEN, (32, 1)), (D.ACT_PER_TOKEN, (200, 40))])
@pytest.mark.parametrize("n,k", [(768, 768), (768, 3072)])
def test_static_matches_linear_forward(hip, mode, ms, n, k):
    ctx = D.Context(0)
    stream = C.c_void_p()
    _lib.check(_lib.lib().tkv_hip_ctx_get_stream(ctx.handle, C.byref(stream)))
    w = O.gi_noise(n * k, 41, 0.02)
    b = O.gi_noise(n, 42, 0.01)
    dw, db = D.DeviceBuffer.from_host(ctx, w), D.DeviceBuffer.from_host(ctx, b)
    lin = D.QuantizedLinear.from_float(ctx, dw, n, k, db, D.WEIGHT_INT8)
    for i, m in enumerate(ms):
        say(f"static linear mode={mode} call {i}: {m}x{n}x{k}")
        x = O.gi_noise(m * k, 43 + i, 1.0 + i)
        dx = D.DeviceBuffer.from_host(ctx, x)
        dy_ref = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        lin.forward(dx, m, dy_ref, mode)
        ctx.synchronize()
        rc = _static(lin, dx, m, mode, dy, stream)
        assert rc == _lib.OK, _lib.last_error() if hasattr(_lib, "last_error") else rc
        ctx.synchronize()
        want, got = dy_ref.download(), dy.download()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (mode, m, n, k)
        for buf in (dx, dy_ref, dy):
            buf.close()
    lin.close()
    dw.close()
    db.close()
    ctx.close()


def test_static_single_pass_quantize_across_slot_reset(hip):
    """Per-tensor activations of 8192 x 3072 take the single-pass calibrate +
    quantize kernel, whose grid barrier runs on the static area's slots; an
    m <= 32 per-tensor call in between clears those slots with the split-K
    sums.  Three calls in a row (large, small, large), each bit-exact against
    tkv_hip_linear_forward."""
    ctx = D.Context(0)
    stream = C.c_void_p()
    _lib.check(_lib.lib().tkv_hip_ctx_get_stream(ctx.handle, C.byref(stream)))
    n, k = 768, 3072
    w = O.gi_noise(n * k, 45, 0.02)
    b = O.gi_noise(n, 46, 0.01)
    dw, db = D.DeviceBuffer.from_host(ctx, w), D.DeviceBuffer.from_host(ctx, b)
    lin = D.QuantizedLinear.from_float(ctx, dw, n, k, db, D.WEIGHT_INT8)
    for i, m in enumerate((8192, 4, 8192)):
        say(f"static linear single-pass sequence call {i}: {m}x{n}x{k}")
        x = O.gi_noise(m * k, 47 + i, 1.0 + i)
        dx = D.DeviceBuffer.from_host(ctx, x)
        dy_ref = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        lin.forward(dx, m, dy_ref, D.ACT_PER_TENSOR)
        ctx.synchronize()
        assert _static(lin, dx, m, D.ACT_PER_TENSOR, dy, stream) == _lib.OK
        ctx.synchronize()
        assert np.array_equal(dy.download().view(np.uint32), dy_ref.download().view(np.uint32)), m
        for buf in (dx, dy_ref, dy):
            buf.close()
    lin.close()
    dw.close()
    db.close()
    ctx.close()


def test_static_refuses_oversize(hip):
    ctx = D.Context(0)
    n, k = 256, 3072
    w = O.gi_noise(n * k, 44, 0.02)
    dw = D.DeviceBuffer.from_host(ctx, w)
    lin = D.QuantizedLinear.from_float(ctx, dw, n, k, None, D.WEIGHT_INT8)
    m = (32 << 20) // k + 1
    dx = D.DeviceBuffer(ctx, 256)
    dy = D.DeviceBuffer(ctx, 256)
    rc = _lib.lib().tkv_hip_linear_forward_static(lin.handle, C.c_void_p(dx.ptr), m, 0,
                                                  C.c_void_p(dy.ptr), None)
    assert rc == _lib.BAD_ARG
    lin.close()
    fp8 = D.QuantizedLinear.from_float(ctx, dw, n, k, None, D.WEIGHT_FP8)
    rc = _lib.lib().tkv_hip_linear_forward_static(fp8.handle, C.c_void_p(dx.ptr), 1, 0,
                                                  C.c_void_p(dy.ptr), None)
    assert rc == _lib.UNSUPPORTED
    fp8.close()
    for buf in (dx, dw, dy):
        buf.close()
    ctx.close()
