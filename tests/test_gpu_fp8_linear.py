"""GPU parity of configs[3]: the FP8-e4m3 W8A8 linear (per-tensor FP8
activations, per-output-channel FP8 weights, FP32 accumulate, per-channel
dequant + bias), through the C ABI, against the oracle's R-ext restatement
(oracle/tkv_oracle.c: tkvo_quantize_fp8_e4m3_dynamic_tensor,
tkvo_fp8_weight_pack, tkvo_matmul_fp8_e4m3_scaled; the scaled extension of
tv/quantization/matmul.tkv:46-66).

Bars:
* codes (raw e4m3 bytes) and scales (f32 bits): bit-exact;
* outputs: the exact product sum S of the reference's decoder, then
  y_ref = fl32(fl64(fl64(S * sa) * sw[n]) + b[n]).  With the scale
  s = sa * sw[n] and sum_k |p_k| the reference products' magnitude sum,
    reference-products path (f16 MFMA):
        |y - y_ref| <= s * 8 * 2^-24 * sum|p| + 2 ulp(y_ref) + 2^-50 (s sum|p| + |b|)
    full-rate path (FP8 MFMA, hardware OCP decode, reduced-precision sums):
        |y - y_ref| <= s * (2^-10 * sum|p_ocp| + sum|p_ocp - p_ref|) + (same terms)
  where p_ocp are the products of the OCP decode: a subnormal code reads
  twice the reference decoder's value, so sum|p_ocp - p_ref| is the exact
  subnormal deviation (0 when no operand code is subnormal).
The exact S is a float64 matrix product of decoded codes: every product is
a multiple of 2^-20 below 2^18, so every partial sum is exact in f64 for
K < 2^15 whatever the summation order; sampled rows are checked against the
oracle's own scalar function bit for bit.
"""
import ctypes as C
import functools
import sys

import numpy as np
import pytest

import oracle as O
from tokenvector.inference_amd import _lib
from tokenvector.inference_amd import device as D

pytestmark = pytest.mark.gpu

SHAPES = [("qkv", 2304, 768), ("attn_out", 768, 768), ("mlp_up", 3072, 768),
          ("mlp_down", 768, 3072)]
FORMATS = [(D.WEIGHT_FP8, "reference_products"), (D.WEIGHT_FP8_FAST, "fast")]
RNG = np.random.default_rng(20261202)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx(hip):
    c = D.Context(0)
    yield c
    c.close()


def _d2h(ctx, ptr, shape, dtype):
    out = np.empty(shape, dtype)
    _lib.check(_lib.lib().tkv_hip_memcpy_d2h(ctx.handle, out.ctypes.data_as(C.c_void_p),
                                             C.c_void_p(ptr), out.nbytes))
    return out


def _dec_tables():
    """(reference decoder, OCP decoder) values of the 256 raw bytes, f64.
    The reference table is the oracle's (pinned exhaustively); the OCP one
    differs only on subnormal codes (twice the reference's value)."""
    ref = O.dequantize_fp8_e4m3(np.arange(256, dtype=np.int32) - 128).astype(np.float64)
    ocp = ref.copy()
    sub = (((np.arange(256) >> 3) & 15) == 0) & ((np.arange(256) & 7) != 0)
    ocp[sub] *= 2.0
    return ref, ocp


REF_DEC, OCP_DEC = _dec_tables()


@functools.lru_cache(maxsize=2)
def _activation(m, k):
    """configs[3] activations N(0, 1) (seed 0 for K = 768, seed 7 for
    K = 3072, as the bench) and their oracle FP8 pack (codes [m, k], scale)."""
    x = O.gi_noise(m * k, 0 if k == 768 else 7, 1.0)
    codes, s = O.quantize_fp8_e4m3_dynamic_tensor(x)
    return x, codes.reshape(m, k), s


def _inputs(n, k, m, j):
    """configs[3] inputs: configs[2]'s layer-0 weight / bias seeds."""
    w = O.gi_noise(n * k, 10 + j + 1, 0.02)
    b = O.gi_noise(n, 10 + j + 51, 0.01)
    return _activation(m, k)[0], w, b


def _expected(a_codes, w_codes, sa, sw, b, rows, fast):
    """y_ref and the stated tolerance on the given rows (int32 offset codes)."""
    ai = a_codes[rows] + 128
    wi = w_codes + 128
    da, dw = REF_DEC[ai], REF_DEC[wi]
    s = da @ dw.T                                     # exact (see module docstring)
    asum = np.abs(da) @ np.abs(dw).T
    scale = np.float64(sa) * sw.astype(np.float64)[None, :]
    y_ref = ((s * np.float64(sa)) * sw.astype(np.float64)[None, :]
             + b.astype(np.float64)[None, :]).astype(np.float32)
    if fast:
        asum_ocp = np.abs(OCP_DEC[ai]) @ np.abs(OCP_DEC[wi]).T
        delta = 2.0 ** -10 * asum_ocp + (asum_ocp - asum) + 1e-12 * asum_ocp
        mag = scale * asum_ocp + np.abs(b.astype(np.float64))[None, :]
    else:
        delta = 8 * 2.0 ** -24 * asum
        mag = scale * asum + np.abs(b.astype(np.float64))[None, :]
    ulp = np.spacing(np.abs(y_ref)).astype(np.float64)
    tol = scale * delta * (1 + 1e-9) + 2 * ulp + 2.0 ** -50 * mag
    return y_ref, tol


@pytest.mark.parametrize("fmt,name", FORMATS)
@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_fp8_weight_pack(ctx, fmt, name, shape):
    """tkv_hip_weight_create(FP8 / FP8_FAST): per-channel scales and e4m3
    codes bit-exact (rows zero padded to the GEMM stride)."""
    _, n, k = shape
    j = [s[0] for s in SHAPES].index(shape[0])
    say(f"fp8 weight pack {shape[0]} {n}x{k} fmt={name}")
    _, w, b = _inputs(n, k, 1, j)
    dw, db = D.DeviceBuffer.from_host(ctx, w), D.DeviceBuffer.from_host(ctx, b)
    lin = D.QuantizedLinear.from_float(ctx, dw, n, k, db, fmt)
    assert lin.format == fmt and lin.n == n and lin.k % 128 == 0
    codes = _d2h(ctx, lin.codes, (n, lin.k), np.uint8)
    scales = _d2h(ctx, lin.scales, (n,), np.float32)
    bias = _d2h(ctx, lin.bias, (n,), np.float32)
    oc, osc = O.fp8_weight_pack(w, n, k)
    assert np.array_equal(scales.view(np.uint32), osc.view(np.uint32))
    assert np.array_equal(codes[:, :k], (oc.reshape(n, k) + 128).astype(np.uint8))
    assert np.all(codes[:, k:] == 0)
    assert np.array_equal(bias.view(np.uint32), b.view(np.uint32))
    sub = int(np.sum((((codes[:, :k] >> 3) & 15) == 0) & ((codes[:, :k] & 7) != 0)))
    say(f"  subnormal weight codes: {sub}")
    lin.close()


@pytest.mark.parametrize("m", [2048, 8192, 32768])
@pytest.mark.parametrize("k", [768, 3072])
def test_fp8_act_quantize(ctx, m, k):
    """Per-tensor FP8 activation pack on device (scale = max|x| / 240, no
    host sync between calibration and encode): codes and scale bit-exact."""
    say(f"fp8 activation pack {m}x{k}")
    x, oc, os_ = _activation(m, k)
    dx = D.DeviceBuffer.from_host(ctx, x)
    q = D.DeviceBuffer.empty(ctx, m * k, np.uint8)
    p = D.params_buffer(ctx)
    D.quantize_fp8_e4m3_dynamic_tensor(ctx, dx, m * k, q, p)
    got = q.download()
    prm = D.read_params(p)
    assert np.float32(prm.scale).view(np.uint32) == os_.view(np.uint32)
    assert np.array_equal(got, (oc.reshape(-1) + 128).astype(np.uint8))
    sub = int(np.sum((((got >> 3) & 15) == 0) & ((got & 7) != 0)))
    say(f"  subnormal activation codes: {sub} of {m * k}")
    for buf in (dx, q, p):
        buf.close()


def _check_forward(ctx, shape, fmt, m, sample_rows):
    name, n, k = shape
    j = [s[0] for s in SHAPES].index(name)
    fast = fmt == D.WEIGHT_FP8_FAST
    x, w, b = _inputs(n, k, m, j)
    dx, dw, db = (D.DeviceBuffer.from_host(ctx, v) for v in (x, w, b))
    lin = D.QuantizedLinear.from_float(ctx, dw, n, k, db, fmt)
    dw.close()
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    lin.forward(dx, m, dy, D.ACT_PER_TENSOR)
    y = dy.download().reshape(m, n)
    _, a_codes, sa = _activation(m, k)
    w_codes, sw = O.fp8_weight_pack(w, n, k)
    w_codes = w_codes.reshape(n, k)
    rows = np.arange(m) if sample_rows is None else np.sort(
        RNG.choice(m, sample_rows, replace=False))
    y_ref, tol = _expected(a_codes, w_codes, sa, sw, b, rows, fast)
    # the f64 matrix product above equals the oracle's scalar function
    chk = rows[:: max(1, len(rows) // 3)][:3]
    oy = O.matmul_fp8_e4m3_scaled(a_codes[chk], w_codes, b, len(chk), n, k, sa, sw)
    sel = np.searchsorted(rows, chk)
    assert np.array_equal(oy.reshape(len(chk), n).view(np.uint32), y_ref[sel].view(np.uint32))
    err = np.abs(y[rows].astype(np.float64) - y_ref.astype(np.float64))
    ratio = float(np.max(err / tol))
    say(f"  {name} m={m} {'fast' if fast else 'ref'}: max err / tol = {ratio:.3g}, "
        f"max |err| = {float(err.max()):.3g}")
    assert np.all(err <= tol), ratio
    for buf in (dx, db, dy):
        buf.close()
    lin.close()


@pytest.mark.parametrize("fmt,name", FORMATS)
@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_fp8_linear_forward_m2048(ctx, fmt, name, shape):
    """weight_create(FP8 / FP8_FAST) + linear_forward(ACT_PER_TENSOR) at
    M = 2048, every output against the exact sum."""
    say(f"fp8 linear {shape[0]} M=2048 {name}")
    _check_forward(ctx, shape, fmt, 2048, None)


@pytest.mark.parametrize("m", [8192, 32768])
@pytest.mark.parametrize("fmt,name", FORMATS)
@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_fp8_linear_forward_large(ctx, fmt, name, shape, m):
    """The same at M = 8192 and 32768 on 192 sampled rows (the activation
    scale and codes still come from the whole tensor)."""
    say(f"fp8 linear {shape[0]} M={m} {name} (192 sampled rows)")
    _check_forward(ctx, shape, fmt, m, 192)


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("per_token", [False, True])
def test_fp8_gemm_scaled_all_codes(ctx, fast, per_token):
    """tkv_hip_dev_matmul_fp8_e4m3{,_fast} with real scale pointers on codes
    drawn from every finite e4m3 byte (a quarter of them subnormal-heavy
    rows), per-tensor and per-token activation scales."""
    m, n, k = 300, 520, 768
    say(f"fp8 scaled gemm all codes fast={fast} per_token={per_token}")
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F])
    subs = np.array([c for c in codes if ((c >> 3) & 15) == 0])
    a = RNG.choice(codes, (m, k))
    a[: m // 4] = RNG.choice(subs, (m // 4, k))
    w = RNG.choice(codes, (n, k))
    w[::5] = RNG.choice(subs, (len(range(0, n, 5)), k))
    sa = RNG.uniform(0.001, 0.05, m if per_token else 1).astype(np.float32)
    sw = RNG.uniform(1e-4, 3e-4, n).astype(np.float32)
    b = RNG.normal(0, 0.01, n).astype(np.float32)
    da = D.DeviceBuffer.from_host(ctx, a.astype(np.uint8))
    dw = D.DeviceBuffer.from_host(ctx, w.astype(np.uint8))
    dsa, dsw, db = (D.DeviceBuffer.from_host(ctx, v) for v in (sa, sw, b))
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    D.matmul_fp8_e4m3(ctx, da, dw, m, n, k, dsa, 1 if per_token else 0, dsw, db, dy, fast=fast)
    y = dy.download().reshape(m, n).astype(np.float64)
    a32, w32 = (a - 128).astype(np.int32), (w - 128).astype(np.int32)
    want = O.matmul_fp8_e4m3_scaled(a32, w32, b, m, n, k, sa, sw, per_token).reshape(m, n)
    ai, wi = a, w
    s_rows = sa.astype(np.float64) if per_token else np.full(m, np.float64(sa[0]))
    scale = s_rows[:, None] * sw.astype(np.float64)[None, :]
    asum = np.abs(REF_DEC[ai]) @ np.abs(REF_DEC[wi]).T
    if fast:
        asum_ocp = np.abs(OCP_DEC[ai]) @ np.abs(OCP_DEC[wi]).T
        delta = 2.0 ** -10 * asum_ocp + (asum_ocp - asum) + 1e-12 * asum_ocp
        mag = scale * asum_ocp
    else:
        delta = 8 * 2.0 ** -24 * asum
        mag = scale * asum
    tol = scale * delta * (1 + 1e-9) + 2 * np.spacing(np.abs(want)).astype(np.float64) \
        + 2.0 ** -50 * (mag + np.abs(b.astype(np.float64))[None, :])
    err = np.abs(y - want.astype(np.float64))
    say(f"  max err / tol = {float(np.max(err / tol)):.3g}")
    assert np.all(err <= tol), float(np.max(err / tol))
    for buf in (da, dw, dsa, dsw, db, dy):
        buf.close()
