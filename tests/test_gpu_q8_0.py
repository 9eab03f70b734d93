"""GPU parity for GGUF Q8_0 weights on the INT8 GEMM (an extension: the
reference decodes Q8_0 blocks to f32, tv/format/gguf.tkv:284-290, and has no
quantized GEMM for them): libtkv_hip through its C ABI against the CPU
oracle's tkvo_matmul_q8_0 on the same seeded inputs.

Bar: unpacked codes and group scales bit-exact against the blocks' bytes and
the reference's f16 decode; the GEMM bit-exact against the oracle (its group
chain is fixed: one fma per group, in group order), on ragged shapes, per
tensor and per token, with and without bias, through the raw GEMM entry and
through tkv_hip_linear_forward; against the reference's decode-then-multiply
of the float activation, within the bound the header states; decode batches
(M <= 32, per-token) through their one-kernel path, bit-exact against the
oracle and against the tile GEMM on the same codes.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle as O
from tokenvector.inference_amd import _lib
from tokenvector.inference_amd import device as D

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(8080)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _bits_equal(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    if a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def _fetch(ctx, ptr, shape, dtype):
    """Copy of device memory owned by a weight handle."""
    out = np.empty(shape, dtype)
    _lib.check(_lib.lib().tkv_hip_memcpy_d2h(ctx.handle, out.ctypes.data_as(C.c_void_p),
                                             C.c_void_p(ptr), out.nbytes))
    return out


def _blocks(n, k, seed, d_lo=0x1C00, d_hi=0x2C00):
    """Raw Q8_0 bytes [n rows x k / 32 blocks]: random codes, f16 scales with
    codes in [d_lo, d_hi) and random sign."""
    r = np.random.default_rng(seed)
    kb = k // 32
    d_codes = r.integers(d_lo, d_hi, (n, kb)) | (r.integers(0, 2, (n, kb)) << 15)
    q = r.integers(-128, 128, (n, k)).astype(np.int8)
    raw = np.zeros((n, kb, 34), np.uint8)
    raw[:, :, 0] = d_codes & 255
    raw[:, :, 1] = (d_codes >> 8) & 255
    raw[:, :, 2:] = q.reshape(n, kb, 32).view(np.uint8)
    return raw.reshape(-1), q, d_codes


@pytest.fixture(scope="module")
def ctx(hip):
    c = D.Context(0)
    yield c
    c.close()


def _weight(ctx, raw, n, k, bias=None):
    dr = D.DeviceBuffer.from_host(ctx, raw)
    db = None if bias is None else D.DeviceBuffer.from_host(ctx, bias)
    wt = D.QuantizedLinear.from_gguf_q8_0(ctx, dr, n, k, db)
    dr.close()
    return wt, db


@pytest.mark.parametrize("n,k", [(1, 32), (5, 96), (64, 768), (300, 3072)])
def test_q8_0_unpack(ctx, n, k):
    """Codes and group scales of the handle: the blocks' int8 bytes and the
    reference decoder's f16 value (every sign, subnormal, inf and NaN code in
    the scale position); rows zero padded to the 128-byte stride, padding
    groups 0."""
    say(f"q8_0 unpack n={n} k={k}")
    raw, q, d_codes = _blocks(n, k, 10 + n)
    kb = k // 32
    d_codes = (np.arange(n * kb, dtype=np.int64) * 257 % 65536).reshape(n, kb)
    raw.reshape(n, kb, 34)[:, :, 0] = d_codes & 255
    raw.reshape(n, kb, 34)[:, :, 1] = d_codes >> 8
    wt, _ = _weight(ctx, raw, n, k)
    assert wt.format == D.WEIGHT_Q8_0
    ldk = wt.k
    assert ldk % 128 == 0 and ldk >= k
    codes = _fetch(ctx, wt.codes, (n, ldk), np.int8)
    gs = _fetch(ctx, wt.scales, (n, ldk // 32), np.float32)
    assert np.array_equal(codes[:, :k], q) and np.all(codes[:, k:] == 0)
    want = np.array([[O.f16_to_f32(int(h)) for h in row] for row in d_codes], np.float32)
    assert _bits_equal(gs[:, :kb], want)
    assert np.all(gs[:, kb:] == 0)
    wt.close()


GEMM_CASES = [(1, 1, 128), (37, 50, 256), (130, 300, 384), (257, 129, 640), (128, 128, 128),
              (1000, 70, 1024)]


@pytest.mark.parametrize("m,n,k", GEMM_CASES)
def test_q8_0_matmul_device(ctx, m, n, k):
    """The raw GEMM entry on ragged shapes (partial tiles in M and N), per
    tensor and per token, with and without bias, bit-exact."""
    say(f"q8_0 gemm m={m} n={n} k={k}")
    raw, q, d_codes = _blocks(n, k, 100 + m + n + k)
    a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    bias = RNG.standard_normal(n).astype(np.float32)
    wt, db = _weight(ctx, raw, n, k, bias)
    assert wt.k == k
    da = D.DeviceBuffer.from_host(ctx, a)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    for sa in (np.array([0.0213], np.float32), (RNG.random(m) * 0.05 + 1e-3).astype(np.float32)):
        ds = D.DeviceBuffer.from_host(ctx, sa)
        stride = 0 if sa.size == 1 else 1
        for b in (db, None):
            D.matmul_q8_0(ctx, da, wt.codes, wt.scales, m, n, k, ds, stride, b, dy)
            want = O.matmul_q8_0(a, raw, sa, m, n, k, None if b is None else bias)
            assert _bits_equal(dy.download(), want), (m, n, k, sa.size, b is None)
        ds.close()
    for buf in (da, dy, db):
        buf.close()
    wt.close()


def test_q8_0_matmul_persistent_tiles(ctx):
    """More tiles than resident workgroups (2304 x 4096: 1152 tiles of 64 x
    128 against 768 resident), so workgroups run several tiles; 96 sampled
    rows bit-exact."""
    m, n, k = 2304, 4096, 256
    say(f"q8_0 gemm persistent m={m} n={n} k={k}")
    raw, q, _ = _blocks(n, k, 77)
    a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    sa = (RNG.random(m) * 0.05 + 1e-3).astype(np.float32)
    wt, _ = _weight(ctx, raw, n, k)
    da = D.DeviceBuffer.from_host(ctx, a)
    ds = D.DeviceBuffer.from_host(ctx, sa)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    D.matmul_q8_0(ctx, da, wt.codes, wt.scales, m, n, k, ds, 1, None, dy)
    got = dy.download()
    rows = np.sort(RNG.choice(m, 96, replace=False))
    want = O.matmul_q8_0(a[rows], raw, sa[rows], rows.size, n, k)
    assert _bits_equal(got[rows], want)
    for buf in (da, ds, dy):
        buf.close()
    wt.close()


def test_q8_0_special_scales(ctx):
    """Zero, subnormal, negative, inf and NaN group scales: outputs bit-exact,
    NaN where the oracle's is NaN."""
    m, n, k = 40, 64, 256
    raw, q, _ = _blocks(n, k, 5)
    kb = k // 32
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8001, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00,
                         0x7E00, 0x3C00, 0xBC00], np.int64)
    d_codes = specials[np.arange(n * kb) % specials.size].reshape(n, kb)
    raw.reshape(n, kb, 34)[:, :, 0] = d_codes & 255
    raw.reshape(n, kb, 34)[:, :, 1] = d_codes >> 8
    a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    sa = np.array([1e-3], np.float32)
    wt, _ = _weight(ctx, raw, n, k)
    da = D.DeviceBuffer.from_host(ctx, a)
    ds = D.DeviceBuffer.from_host(ctx, sa)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    D.matmul_q8_0(ctx, da, wt.codes, wt.scales, m, n, k, ds, 0, None, dy)
    assert _bits_equal(dy.download(), O.matmul_q8_0(a, raw, sa, m, n, k))
    for buf in (da, ds, dy):
        buf.close()
    wt.close()


@pytest.mark.parametrize("m,n,k", [(33, 200, 256), (512, 2304, 768), (8192, 768, 3072)])
@pytest.mark.parametrize("act", [D.ACT_PER_TENSOR, D.ACT_PER_TOKEN])
def test_q8_0_linear_forward(ctx, m, n, k, act):
    """tkv_hip_linear_forward on a Q8_0 handle: the activation quantized by the
    INT8 path (calibrate_minmax + quantize_int8_symmetric per tensor,
    quantize_dynamic_int8_rowwise per token), then the Q8_0 GEMM; sampled rows
    bit-exact against the oracle's quantizer + tkvo_matmul_q8_0, and every
    output within the stated bound of the reference's decode-then-multiply of
    x (dequantize_gguf, f64 matmul)."""
    say(f"q8_0 linear_forward m={m} n={n} k={k} act={act}")
    raw, q, d_codes = _blocks(n, k, 300 + n)
    x = O.gi_noise(m * k, 5 + m, 1.0).reshape(m, k)
    bias = O.gi_noise(n, 9, 0.01)
    wt, db = _weight(ctx, raw, n, k, bias)
    dx = D.DeviceBuffer.from_host(ctx, x)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    wt.forward(dx, m, dy, act)
    got = dy.download()
    if act == D.ACT_PER_TENSOR:
        p = O.calibrate_minmax(x.reshape(-1), 1)
        codes = np.asarray(O.quantize_int8_symmetric(x.reshape(-1), p.scale), np.int32).reshape(m, k)
        sa = np.full(m, p.scale, np.float32)
        sa_arg = np.array([p.scale], np.float32)
    else:
        c, s = O.quantize_dynamic_int8_rowwise(x.reshape(-1), m, k)
        codes = np.asarray(c, np.int32).reshape(m, k)
        sa = np.asarray(s, np.float32)
        sa_arg = sa
    rows = np.arange(m) if m <= 64 else np.sort(RNG.choice(m, 48, replace=False))
    want = O.matmul_q8_0(codes[rows], raw, sa_arg if sa_arg.size == 1 else sa_arg[rows],
                         rows.size, n, k, bias)
    assert _bits_equal(got[rows], want)
    # the reference's semantics: decode the blocks to f32, multiply the float x
    w = O.dequantize_gguf(raw, n * k, O.GGUF_Q8_0).reshape(n, k).astype(np.float64)
    ref = x[rows].astype(np.float64) @ w.T + bias.astype(np.float64)
    kb = k // 32
    d = np.abs(d_codes.astype(np.uint16).view(np.float16).astype(np.float64))
    absw = np.abs(w).sum(axis=1)
    chain = kb * 2.0 ** -24 * 127 * (d * np.abs(q.astype(np.float64)).reshape(n, kb, 32).sum(axis=2)).sum(axis=1)
    s = sa[rows].astype(np.float64)[:, None]
    # activation codes + group chain, then the epilogue's roundings
    bound = ((s / 2 + 2.0 ** -17 * s) * absw[None] + chain[None] * s) * (1 + 2.0 ** -20) \
        + 2.0 ** -23 * np.abs(ref)
    err = np.abs(got[rows].astype(np.float64) - ref)
    assert np.all(err <= bound), float((err / bound).max())
    for buf in (dx, dy, db):
        buf.close()
    wt.close()


def test_q8_0_errors(ctx, hip):
    """K % 32 != 0 at creation: BAD_ARG (ValueError); K not a multiple of
    128 at forward or in the raw GEMM: UNSUPPORTED; the no-allocation entry
    point takes INT8 weights only."""
    raw, _, _ = _blocks(4, 96, 3)
    dr = D.DeviceBuffer.from_host(ctx, raw)
    with pytest.raises(ValueError):
        D.QuantizedLinear.from_gguf_q8_0(ctx, dr, 4, 80)
    wt = D.QuantizedLinear.from_gguf_q8_0(ctx, dr, 4, 96)
    dx = D.DeviceBuffer.empty(ctx, (2, 96), np.float32)
    dy = D.DeviceBuffer.empty(ctx, (2, 4), np.float32)
    with pytest.raises(_lib.TkvHipError):
        wt.forward(dx, 2, dy)
    rc = _lib.lib().tkv_hip_linear_forward_static(wt.handle, D._vp(dx), 2, 0, D._vp(dy), None)
    assert rc == _lib.UNSUPPORTED
    ds = D.DeviceBuffer.from_host(ctx, np.ones(1, np.float32))
    da = D.DeviceBuffer.empty(ctx, (2, 96), np.int8)
    with pytest.raises(_lib.TkvHipError):
        D.matmul_q8_0(ctx, da, wt.codes, wt.scales, 2, 4, 96, ds, 0, None, dy)
    with pytest.raises(ValueError):
        D.matmul_q8_0(ctx, da, wt.codes, wt.scales, 2, 4, 128, ds, 2, None, dy)   # stride 2
    for buf in (dr, dx, dy, ds, da):
        buf.close()
    wt.close()


Q8_DECODE = [(1, 2304, 768), (4, 768, 3072), (5, 100, 192), (16, 3072, 768), (17, 768, 3072),
             (32, 2304, 768), (32, 768, 3072)]


@pytest.mark.parametrize("dma", [None, 0, 1])
@pytest.mark.parametrize("m,n,k", Q8_DECODE)
def test_q8_0_decode(ctx, m, n, k, dma):
    """Decode batches (M <= 32, per-token activations) take the one-kernel
    Q8_0 decode path (in-kernel per-token quantize, one MFMA per group, the
    group chain in LDS), with the weight path automatic or forced (registers,
    or whole lines through LDS; 4 DMAs per wave at K = 192): bit-exact
    against the oracle's rowwise quantizer + tkvo_matmul_q8_0, and the same
    bits as the tile GEMM on those codes."""
    say(f"q8_0 decode m={m} n={n} k={k} dma={dma}")
    raw, q, _ = _blocks(n, k, 900 + m + n)
    x = O.gi_noise(m * k, 50 + m, 1.0).reshape(m, k)
    bias = O.gi_noise(n, 51, 0.01)
    wt, db = _weight(ctx, raw, n, k, bias)
    dx = D.DeviceBuffer.from_host(ctx, x)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    ctx.set_tuning(D.TUNE_DECODE_DMA, -1 if dma is None else dma)
    try:
        wt.forward(dx, m, dy, D.ACT_PER_TOKEN)
    finally:
        ctx.set_tuning(D.TUNE_DECODE_DMA, -1)
    got = dy.download()
    c, s = O.quantize_dynamic_int8_rowwise(x.reshape(-1), m, k)
    codes = np.asarray(c, np.int32).reshape(m, k)
    sa = np.asarray(s, np.float32)
    assert _bits_equal(got, O.matmul_q8_0(codes, raw, sa, m, n, k, bias))
    if k % 128 == 0:
        da = D.DeviceBuffer.from_host(ctx, codes.astype(np.int8))
        ds = D.DeviceBuffer.from_host(ctx, sa)
        dy2 = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        D.matmul_q8_0(ctx, da, wt.codes, wt.scales, m, n, k, ds, 1, db, dy2)
        assert _bits_equal(dy2.download(), got)
        for buf in (da, ds, dy2):
            buf.close()
    for buf in (dx, dy, db):
        buf.close()
    wt.close()


@pytest.mark.parametrize("group", [1, 3, 16])
def test_q8_0_decode_forced_groups(ctx, group):
    """Forced tokens per workgroup (the context's decode-group override): one
    token, a group that leaves a ragged last group, and 16 (the largest LDS
    footprint, capped by the device's LDS per workgroup) stay bit-exact."""
    m, n, k = 32, 768, 3072
    say(f"q8_0 decode forced group={group}")
    raw, q, _ = _blocks(n, k, 1234)
    x = O.gi_noise(m * k, 77, 1.0).reshape(m, k)
    wt, _ = _weight(ctx, raw, n, k)
    dx = D.DeviceBuffer.from_host(ctx, x)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    ctx.set_tuning(D.TUNE_DECODE_GROUP, group)
    try:
        wt.forward(dx, m, dy, D.ACT_PER_TOKEN)
        got = dy.download()
    finally:
        ctx.set_tuning(D.TUNE_DECODE_GROUP, -1)
    c, s = O.quantize_dynamic_int8_rowwise(x.reshape(-1), m, k)
    want = O.matmul_q8_0(np.asarray(c, np.int32).reshape(m, k), raw, np.asarray(s, np.float32),
                         m, n, k)
    assert _bits_equal(got, want)
    for buf in (dx, dy):
        buf.close()
    wt.close()
