"""GPU parity at full size against the committed golden digests.

tests/golden/w8a8_pipeline.json holds SHA-256 digests of every stage of the
W8A8 pipeline on the benchmark's seeded inputs. Covered are config 1
(1024x3072x768) and the four GPT-2-124M linears at M = 8192. The device path
(tkv_hip_weight_create, tkv_hip_dev_calibrate_minmax,
tkv_hip_dev_quantize_int8_tensor, tkv_hip_dev_quantize_dynamic_int8_rowwise,
tkv_hip_linear_forward) must reproduce every digest bit for bit. The host
only generates the inputs; no GEMM is recomputed here.
"""
import ctypes as C
import hashlib
import json
import os
import sys

import numpy as np
import pytest

import oracle as O
from tokenvector.inference_amd import _lib
from tokenvector.inference_amd import device as D

pytestmark = pytest.mark.gpu

with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                       "w8a8_pipeline.json")) as _f:
    PIPE = json.load(_f)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _d2h(ctx, ptr, shape, dtype):
    out = np.empty(shape, dtype)
    _lib.check(_lib.lib().tkv_hip_memcpy_d2h(ctx.handle, out.ctypes.data_as(C.c_void_p),
                                             C.c_void_p(ptr), out.nbytes))
    return out


@pytest.fixture(scope="module")
def ctx(hip):
    c = D.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("case", PIPE["cases"], ids=[c["name"] for c in PIPE["cases"]])
def test_w8a8_pipeline_matches_golden(ctx, case):
    m, n, k, s = case["m"], case["n"], case["k"], case["seeds"]
    print(f"golden {case['name']} m={m} n={n} k={k}", flush=True)
    sys.stdout.flush()
    x = O.gi_noise(m * k, s["x"], case["sigma"]["x"])
    w = O.gi_noise(n * k, s["w"], case["sigma"]["w"])
    b = O.gi_noise(n, s["bias"], case["sigma"]["bias"])
    dx, dw, db = (D.DeviceBuffer.from_host(ctx, v) for v in (x, w, b))

    lin = D.QuantizedLinear.from_float(ctx, dw, n, k, db, D.WEIGHT_INT8)
    ldk = lin.k
    assert ldk >= k and lin.n == n
    codes = _d2h(ctx, lin.codes, (n, ldk), np.int8)
    assert not codes[:, k:].any()
    assert _sha(codes[:, :k]) == case["w_codes_sha256"]
    assert _sha(_d2h(ctx, lin.scales, (n,), np.float32)) == case["w_scales_sha256"]

    params = D.params_buffer(ctx)
    D.calibrate_minmax(ctx, dx, m * k, 1, params)
    q = D.DeviceBuffer.empty(ctx, (m, k), np.int8)
    D.quantize_int8_tensor(ctx, dx, m * k, params, q)
    scale = np.float32(D.read_params(params).scale)
    assert "%08x" % int(scale.view(np.uint32)) == case["x_scale_f32"]
    assert _sha(q.download()) == case["x_codes_sha256"]

    rs = D.DeviceBuffer.empty(ctx, (m,), np.float32)
    D.quantize_dynamic_int8_rowwise(ctx, dx, m, k, q, rs)
    assert _sha(rs.download()) == case["x_row_scales_sha256"]
    assert _sha(q.download()) == case["x_row_codes_sha256"]

    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    lin.forward(dx, m, dy, D.ACT_PER_TENSOR)
    y = dy.download()
    head = ["%08x" % v for v in y.reshape(-1)[:8].view(np.uint32)]
    assert head == case["y_per_tensor_head_f32"]
    assert _sha(y) == case["y_per_tensor_sha256"]
    lin.forward(dx, m, dy, D.ACT_PER_TOKEN)
    assert _sha(dy.download()) == case["y_per_token_sha256"]
    lin.close()
