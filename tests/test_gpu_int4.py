"""GPU parity for grouped INT4 weights (tv/quantization/int4.tkv) and the GGUF
block formats (tv/format/gguf.tkv:284-313): libtkv_hip through its C ABI
against the CPU oracle on the same seeded inputs.

Bar: codes, scales, zero points and dequantized values bit-exact.  The INT4
GEMM accumulates in f64 with exact products, so it may differ from the
reference's sequential sum only by the order of the additions (and, where it
applies each group's scale once to the group's sum of x (nibble - 8), by one
fma rounding per group: gs + K / gs roundings in all, at most 2 K):
|y - y_ref| <= 2 K 2^-53 sum_k |a_k w_k| + ulp(y_ref) per element, and
bit-exact on dyadic inputs, where every partial sum is exact.
"""
import sys

import numpy as np
import pytest

import oracle as O
from tokenvector.inference_amd import _lib
from tokenvector.inference_amd import device as D
from tokenvector.inference_amd import gguf as G
from tokenvector.inference_amd import int4 as I4

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20261202)


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


def _weights(rows, cols, seed):
    w = O.gi_noise(rows * cols, seed, 0.02)
    if w.size > 100:
        w = O.add_outliers(w, 0.001, seed + 1, seed + 2, 0.5)
    return w


@pytest.fixture(scope="module")
def ctx(hip):
    c = D.Context(0)
    yield c
    c.close()


INT4_SHAPES = [(1, 8, 4), (6, 30, 3), (7, 96, 32), (64, 768, 128), (300, 3072, 64), (2304, 768, 32)]


@pytest.mark.parametrize("rows,cols,gs", INT4_SHAPES)
def test_int4_quantize_dequantize(hip, rows, cols, gs):
    """quantize / dequantize, symmetric and AWQ-asym: bit-exact host mirrors
    (int32-per-byte lists, appended scales and zero points)."""
    say(f"int4 quantize {rows}x{cols} gs={gs}")
    w = _weights(rows, cols, 11 + cols)
    pk = np.full(rows * cols // 2 + 3, 77, np.int32)     # longer list: cleared entirely
    scales = []
    I4.quantize_int4_grouped(w, rows, cols, gs, pk, scales)
    opk, osc = O.quantize_int4_grouped(w, rows, cols, gs, npacked=pk.size)
    assert np.array_equal(pk, opk) and _bits_equal(scales, osc)
    y = np.zeros(rows * cols, np.float32)
    I4.dequantize_int4_grouped(pk, y, rows, cols, gs, scales)
    assert _bits_equal(y, O.dequantize_int4_grouped(opk, rows, cols, gs, osc))

    pk = np.zeros(rows * cols // 2, np.int32)
    scales, zps = [], []
    I4.quantize_int4_grouped_asym(w, rows, cols, gs, pk, scales, zps)
    opk, osc, ozp = O.quantize_int4_grouped_asym(w, rows, cols, gs)
    assert np.array_equal(pk, opk) and _bits_equal(scales, osc) and np.array_equal(zps, ozp)
    I4.dequantize_int4_grouped_asym(pk, y, rows, cols, gs, scales, zps)
    assert _bits_equal(y, O.dequantize_int4_grouped_asym(opk, rows, cols, gs, osc, ozp))


def test_int4_special_values_and_errors(hip):
    """NaN / inf / flat / all-positive / all-negative groups, then every
    ValueError case of the .tkv functions."""
    say("int4 special values")
    x = np.array([np.nan, 1.0, 2.0, 3.0,   1.0, np.nan, -2.0, 0.5,   np.inf, 1.0, 0.0, -1.0,
                  3.0, 3.0, 3.0, 3.0,   2.0, 3.0, 4.0, 5.0,   -5.0, -4.0, -3.0, -2.0], np.float32)
    for fn, ofn in ((I4.quantize_int4_grouped, O.quantize_int4_grouped),):
        pk, sc = np.zeros(12, np.int32), []
        fn(x, 1, 24, 4, pk, sc)
        opk, osc = ofn(x, 1, 24, 4)
        assert np.array_equal(pk, opk) and _bits_equal(sc, osc)
    pk, sc, zp = np.zeros(12, np.int32), [], []
    I4.quantize_int4_grouped_asym(x, 1, 24, 4, pk, sc, zp)
    opk, osc, ozp = O.quantize_int4_grouped_asym(x, 1, 24, 4)
    assert np.array_equal(pk, opk) and _bits_equal(sc, osc) and np.array_equal(zp, ozp)
    w = np.ones(16, np.float32)
    with pytest.raises(ValueError):
        I4.quantize_int4_grouped(w, 2, 8, 3, np.zeros(8, np.int32), [])      # cols % gs
    with pytest.raises(ValueError):
        I4.quantize_int4_grouped(w, 1, 7, 7, np.zeros(8, np.int32), [])      # odd cols
    with pytest.raises(ValueError):
        I4.quantize_int4_grouped(w, 3, 8, 4, np.zeros(12, np.int32), [])     # short src
    with pytest.raises(ValueError):
        I4.quantize_int4_grouped(w, 2, 8, 4, np.zeros(7, np.int32), [])      # short packed
    with pytest.raises(ValueError):
        I4.dequantize_int4_grouped(np.zeros(8, np.int32), np.zeros(16, np.float32), 2, 8, 4,
                                   [1.0, 1.0, 1.0])                           # short scales
    with pytest.raises(ValueError):
        I4.dequantize_int4_grouped(np.zeros(8, np.int32), np.zeros(15, np.float32), 2, 8, 4,
                                   [1.0] * 4)                                 # short dst


def test_int4_device_variants(ctx):
    """Device quantize (bytes) / dequantize / permute against the oracle."""
    rows, cols, gs = 768, 3072, 128
    say(f"int4 device {rows}x{cols} gs={gs}")
    w = _weights(rows, cols, 5)
    dw = D.DeviceBuffer.from_host(ctx, w)
    dp = D.DeviceBuffer.empty(ctx, rows * cols // 2, np.uint8)
    ds = D.DeviceBuffer.empty(ctx, rows * cols // gs, np.float32)
    dz = D.DeviceBuffer.empty(ctx, rows * cols // gs, np.int64)
    dy = D.DeviceBuffer.empty(ctx, rows * cols, np.float32)
    D.quantize_int4_grouped(ctx, dw, rows, cols, gs, dp, ds)
    opk, osc = O.quantize_int4_grouped(w, rows, cols, gs)
    assert np.array_equal(dp.download().astype(np.int32), opk) and _bits_equal(ds.download(), osc)
    D.dequantize_int4_grouped(ctx, dp, rows, cols, gs, ds, None, dy)
    assert _bits_equal(dy.download(), O.dequantize_int4_grouped(opk, rows, cols, gs, osc))
    D.quantize_int4_grouped(ctx, dw, rows, cols, gs, dp, ds, dz)
    opk, osc, ozp = O.quantize_int4_grouped_asym(w, rows, cols, gs)
    assert np.array_equal(dp.download().astype(np.int32), opk)
    assert _bits_equal(ds.download(), osc) and np.array_equal(dz.download(), ozp)
    D.dequantize_int4_grouped(ctx, dp, rows, cols, gs, ds, dz, dy)
    assert _bits_equal(dy.download(), O.dequantize_int4_grouped_asym(opk, rows, cols, gs, osc, ozp))
    perm = RNG.permutation(cols).astype(np.int64)
    dperm = D.DeviceBuffer.from_host(ctx, perm)
    for inverse in (False, True):
        D.permute_cols(ctx, dw, rows, cols, dperm, inverse, dy)
        assert np.array_equal(dy.download(), O.permute_cols(w, rows, cols, perm, inverse))


def test_permute_cols_host(hip):
    x = O.gi_noise(5 * 7, 3, 1.0)
    perm = [3, 0, 6, 1, 5, 2, 4]
    assert np.array_equal(I4.permute_cols(x, 5, 7, perm), O.permute_cols(x, 5, 7, perm))
    assert np.array_equal(I4.inv_permute_cols(I4.permute_cols(x, 5, 7, perm), 5, 7, perm), x)
    with pytest.raises(ValueError):
        I4.permute_cols(x, 5, 7, perm[:-1])
    with pytest.raises(ValueError):
        I4.permute_cols(x, 5, 7, perm[:-1] + [7])
    with pytest.raises(_lib.TkvHipError):
        I4.inv_permute_cols(x, 5, 7, [0, 0, 1, 2, 3, 4, 5])   # ordered overwrites: caller's loop


def _gemm_bound(a, pk, sc, bias, m, n, k, gs, yref):
    wd = np.asarray(O.dequantize_int4_grouped(pk, n, k, gs, sc), np.float64).reshape(n, k)
    s = np.abs(np.asarray(a, np.float64).reshape(m, k)) @ np.abs(wd).T
    return 2 * k * 2.0 ** -53 * s.reshape(-1) + np.spacing(np.abs(yref)).astype(np.float64)


# 2 <= M <= 32 with K % 32 == 0 takes the decode kernel (16-column workgroups
# of 8 waves, K split over workgroups when the column blocks are few and the k
# blocks allow one per wave: (32, 130, 512) in 2, (17, 1000, 1024) in 4,
# (16, 200, 256) unsplit); M = 1 takes the single-row kernel
# (one load step per 512 of K, at most 6 per trip: (1, 70, 3600, 8) runs two
# trips, the second with 2 lanes of its second step inside K; (1, 33, 200, 8)
# one part step), and (3, 50, 80, 16), whose K % 32 != 0, the per-column
# kernel, as does every act-order form.  Larger M takes the 64 x 64 tile
# kernel, with K split over workgroups when the tiles are few for the CUs (256
# CUs): (70, 130, 256) in 2, (300, 768, 768) in 4, (128, 768, 3072) in 20 (the
# last split shorter), (100, 60, 522, 18) in 4 on the LDS form (K % 8 != 0),
# (1100, 1100, 256, 16) in 2 with more tiles than CUs; (520, 1040, 128) has too
# few slices and no split (group scales applied per group: gs % 32 == 0), nor
# has a group-scaled launch with 8 tiles per slice of K or more.  K % 32
# != 0 on the register form: (90, 70, 200, 8) unsplit and (100, 60, 520, 8) in
# 4, each ending in a part slice.  The act-order form always takes the LDS
# form.
GEMM_SHAPES = [(1, 100, 64, 32), (2, 64, 128, 32), (5, 37, 96, 32), (16, 200, 256, 64),
               (32, 130, 512, 128), (17, 1000, 1024, 128), (3, 50, 80, 16),
               (70, 130, 256, 64), (33, 2304, 768, 128), (300, 768, 768, 128),
               (129, 768, 3072, 32), (64, 768, 768, 128), (128, 768, 3072, 128),
               (200, 100, 512, 32), (100, 60, 522, 18), (520, 1040, 128, 32),
               (1100, 1100, 256, 16), (90, 70, 200, 8), (100, 60, 520, 8),
               (1, 70, 3600, 8), (1, 33, 200, 8)]


@pytest.mark.parametrize("m,n,k,gs", GEMM_SHAPES)
def test_int4_matmul(hip, m, n, k, gs):
    say(f"int4 matmul {m}x{n}x{k} gs={gs}")
    a = O.gi_noise(m * k, 7 + m, 1.0)
    w = _weights(n, k, 17 + n)
    pk, sc = O.quantize_int4_grouped(w, n, k, gs)
    b = O.gi_noise(n, 19, 0.01)
    for bias in (b, None):
        y = np.zeros(m * n, np.float32)
        I4.matmul_int4_grouped(a, pk, bias, y, m, n, k, gs, sc)
        ref = O.matmul_int4_grouped(a, pk, bias, m, n, k, gs, sc)
        err = np.abs(y.astype(np.float64) - ref)
        assert np.all(err <= _gemm_bound(a, pk, sc, bias, m, n, k, gs, ref)), (m, n, k)
        assert np.mean(y == ref) > 0.999   # order-only differences are rare after rounding
    perm = RNG.permutation(k).astype(np.int64)
    y = np.zeros(m * n, np.float32)
    I4.matmul_int4_grouped_ordered(a, pk, b, y, m, n, k, gs, sc, perm)
    ref = O.matmul_int4_grouped(a, pk, b, m, n, k, gs, sc, perm=perm)
    ap = O.permute_cols(a, m, k, perm)
    assert np.all(np.abs(y.astype(np.float64) - ref) <= _gemm_bound(ap, pk, sc, b, m, n, k, gs, ref))


def test_int4_matmul_k0(hip):
    """K = 0 on every GEMM form (single row, decode, tile kernel, act-order):
    y is the bias (or zero) broadcast over the rows."""
    n, gs = 37, 8
    b = O.gi_noise(n, 23, 0.01)
    for m in (1, 5, 40, 100):
        say(f"int4 matmul K=0 m={m}")
        for bias in (b, None):
            y = np.full(m * n, np.nan, np.float32)
            I4.matmul_int4_grouped(np.zeros(0, np.float32), np.zeros(0, np.int32), bias, y, m, n,
                                   0, gs, np.zeros(0, np.float32))
            want = np.tile(bias if bias is not None else np.zeros(n, np.float32), m)
            assert np.array_equal(y, want), m
        y = np.full(m * n, np.nan, np.float32)
        I4.matmul_int4_grouped_ordered(np.zeros(0, np.float32), np.zeros(0, np.int32), b, y, m, n,
                                       0, gs, np.zeros(0, np.float32), np.zeros(0, np.int64))
        assert np.array_equal(y, np.tile(b, m)), m


def test_int4_matmul_dyadic_exact_and_errors(hip):
    """Dyadic inputs (40 x 72 x 256: K split in 2 over the tile kernel's
    workgroups; 520 x 72 x 128: unsplit, group scales applied per group):
    every partial sum exact, so the GPU result is the reference's bit for
    bit; then the ValueError / unsupported cases."""
    for m, n, k, gs in ((520, 72, 128, 32), (40, 72, 256, 32)):
        say(f"int4 matmul dyadic {m}x{n}x{k}")
        a = (RNG.integers(-64, 64, m * k) / 16.0).astype(np.float32)
        pk = RNG.integers(0, 256, n * k // 2).astype(np.int32)
        sc = (2.0 ** -RNG.integers(1, 6, n * k // gs)).astype(np.float32)
        b = (RNG.integers(-8, 8, n) / 8.0).astype(np.float32)
        y = np.zeros(m * n, np.float32)
        I4.matmul_int4_grouped(a, pk, b, y, m, n, k, gs, sc)
        assert np.array_equal(y, O.matmul_int4_grouped(a, pk, b, m, n, k, gs, sc))
    with pytest.raises(ValueError):
        I4.matmul_int4_grouped(a, pk, b, y, m, n, k, gs, sc[:-1])
    with pytest.raises(ValueError):
        I4.matmul_int4_grouped(a, pk, b[:-1], y, m, n, k, gs, sc)
    with pytest.raises(_lib.TkvHipError):
        I4.matmul_int4_grouped(a, pk, b, y, m, n, k, 48, sc)        # K % group_size != 0
    with pytest.raises(_lib.TkvHipError):
        I4.matmul_int4_grouped(a, pk, b, y, m, n, k - 1, 51, sc)    # odd K
    with pytest.raises(_lib.TkvHipError):
        I4.matmul_int4_grouped_ordered(a, pk, b, y, m, n, k, gs, sc, np.full(k, k, np.int64))


@pytest.mark.parametrize("m", [1, 4, 17, 32])
@pytest.mark.parametrize("name,n,k", [("qkv", 2304, 768), ("attn_out", 768, 768),
                                      ("mlp_up", 3072, 768), ("mlp_down", 768, 3072)])
def test_int4_decode_gpt2_shapes(ctx, name, n, k, m):
    """Decode batches on the four GPT-2 shapes (group size 128), device
    buffers: every output within the reordering bound of the oracle, a
    second launch bit-identical (the split-K reduction has a fixed order),
    and the register weight path (the context's decode weight-path knob)
    bit-identical to the default path through LDS."""
    gs = 128
    say(f"int4 decode {name} m={m}")
    a = O.gi_noise(m * k, 31 + m, 1.0)
    w = _weights(n, k, 37)
    pk, sc = O.quantize_int4_grouped(w, n, k, gs)
    b = O.gi_noise(n, 41, 0.01)
    da, db = D.DeviceBuffer.from_host(ctx, a), D.DeviceBuffer.from_host(ctx, b)
    dw = D.DeviceBuffer.from_host(ctx, pk.astype(np.uint8))
    ds = D.DeviceBuffer.from_host(ctx, sc)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    D.matmul_int4_grouped(ctx, da, dw, ds, db, None, dy, m, n, k, gs)
    y = dy.download()
    ref = O.matmul_int4_grouped(a, pk, b, m, n, k, gs, sc)
    assert np.all(np.abs(y.astype(np.float64).reshape(-1) - ref) <=
                  _gemm_bound(a, pk, sc, b, m, n, k, gs, ref))
    for _ in range(2):
        D.matmul_int4_grouped(ctx, da, dw, ds, db, None, dy, m, n, k, gs)
        assert np.array_equal(dy.download(), y)
    ctx.set_tuning(D.TUNE_DECODE_DMA, 0)
    try:
        D.matmul_int4_grouped(ctx, da, dw, ds, db, None, dy, m, n, k, gs)
    finally:
        ctx.set_tuning(D.TUNE_DECODE_DMA, -1)
    assert np.array_equal(dy.download(), y)


def test_graph_replays_int4(ctx):
    """matmul_int4_grouped on device buffers captured in one graph: M = 1
    (single-row kernel), 32 (decode kernel, K split over workgroups with
    arrival counts), 200 (tile kernel, K split + split sum) on a 768 x 3072
    weight and 520 (tile kernel unsplit, group scales per group) on a 256 x
    128 one.  Replays after new activations, with eager calls of other sizes
    between them, give the eager results bit for bit; the eager results are
    within the reordering bound of the oracle."""
    say("graph replays int4")
    cases = []
    for (n, k, gs, ms, seed) in ((768, 3072, 128, (1, 32, 200), 61), (256, 128, 32, (520,), 63)):
        w = _weights(n, k, seed)
        pk, sc = O.quantize_int4_grouped(w, n, k, gs)
        dw = D.DeviceBuffer.from_host(ctx, pk.astype(np.uint8))
        ds = D.DeviceBuffer.from_host(ctx, sc)
        b = O.gi_noise(n, seed + 5, 0.01)
        db = D.DeviceBuffer.from_host(ctx, b)
        for m in ms:
            xs = [O.gi_noise(m * k, seed + 10 * i + m, 1.0) for i in range(2)]
            cases.append((m, n, k, gs, pk, sc, b, dw, ds, db, xs,
                          D.DeviceBuffer.empty(ctx, m * k, np.float32),
                          D.DeviceBuffer.empty(ctx, (m, n), np.float32)))

    def run():
        for (m, n, k, gs, pk, sc, b, dw, ds, db, xs, dx, dy) in cases:
            D.matmul_int4_grouped(ctx, dx, dw, ds, db, None, dy, m, n, k, gs)

    want = []
    for i in range(2):
        for c in cases:
            c[11].upload(c[10][i])
        run()
        ctx.synchronize()
        want.append([c[12].download().tobytes() for c in cases])
    for j, (m, n, k, gs, pk, sc, b, dw, ds, db, xs, dx, dy) in enumerate(cases):
        if m * n * k > 10 ** 8:
            continue
        y = np.frombuffer(want[1][j], np.float32)
        ref = O.matmul_int4_grouped(xs[1], pk, b, m, n, k, gs, sc)
        assert np.all(np.abs(y.astype(np.float64) - ref) <= _gemm_bound(xs[1], pk, sc, b, m, n, k,
                                                                          gs, ref)), m
    # eager calls of other sizes on the same weights and workspaces
    m0, n0, k0, gs0, _, _, _, dw0, ds0, db0 = cases[0][:10]
    ox = D.DeviceBuffer.from_host(ctx, O.gi_noise(64 * k0, 99, 1.0))
    oy = D.DeviceBuffer.empty(ctx, (64, n0), np.float32)
    oy2 = D.DeviceBuffer.empty(ctx, (16, n0), np.float32)

    def other():
        D.matmul_int4_grouped(ctx, ox, dw0, ds0, db0, None, oy, 64, n0, k0, gs0)
        D.matmul_int4_grouped(ctx, ox, dw0, ds0, None, None, oy2, 16, n0, k0, gs0)

    other()
    ctx.synchronize()
    with D.Graph(ctx) as g:
        run()
    for rep in range(2):
        for i in range(2):
            for c in cases:
                c[11].upload(c[10][i])
            other()
            ctx.synchronize()
            for c in cases:
                D.memset(ctx, c[12], 0, c[12].nbytes)
            g.launch()
            ctx.synchronize()
            assert [c[12].download().tobytes() for c in cases] == want[i], (rep, i)
    g.close()
    bufs = {}
    for c in cases:
        for buf in c[7:10] + c[11:13]:
            bufs[id(buf)] = buf
    for buf in list(bufs.values()) + [ox, oy, oy2]:
        buf.close()


def test_int4_decode_dyadic_exact(hip):
    """Dyadic inputs through the decode kernel with a K split over
    workgroups: every partial sum is exact, so the result is the reference's
    bit for bit."""
    for m, n, k, gs in ((32, 72, 512, 32), (9, 40, 256, 64)):
        say(f"int4 decode dyadic {m}x{n}x{k}")
        a = (RNG.integers(-64, 64, m * k) / 16.0).astype(np.float32)
        pk = RNG.integers(0, 256, n * k // 2).astype(np.int32)
        sc = (2.0 ** -RNG.integers(1, 6, n * k // gs)).astype(np.float32)
        b = (RNG.integers(-8, 8, n) / 8.0).astype(np.float32)
        y = np.zeros(m * n, np.float32)
        I4.matmul_int4_grouped(a, pk, b, y, m, n, k, gs, sc)
        assert np.array_equal(y, O.matmul_int4_grouped(a, pk, b, m, n, k, gs, sc))


def test_int4_matmul_gpt2_full_size_rows(ctx):
    """GPT-2 mlp-up at M = 8192 on device buffers; sampled rows against the
    oracle (rows are independent), all rows against the same rows recomputed
    in a second launch (deterministic)."""
    m, n, k, gs = 8192, 3072, 768, 128
    say(f"int4 matmul full {m}x{n}x{k}")
    a = O.gi_noise(m * k, 0, 1.0)
    w = _weights(n, k, 23)
    pk, sc = O.quantize_int4_grouped(w, n, k, gs)
    b = O.gi_noise(n, 29, 0.01)
    da, db = D.DeviceBuffer.from_host(ctx, a), D.DeviceBuffer.from_host(ctx, b)
    dw = D.DeviceBuffer.from_host(ctx, pk.astype(np.uint8))
    ds = D.DeviceBuffer.from_host(ctx, sc)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    D.matmul_int4_grouped(ctx, da, dw, ds, db, None, dy, m, n, k, gs)
    y = dy.download()
    rows = np.array([0, 1, 63, 64, 4095, 8191])
    sub = a.reshape(m, k)[rows].reshape(-1)
    ref = O.matmul_int4_grouped(sub, pk, b, rows.size, n, k, gs, sc)
    got = y[rows].reshape(-1)
    assert np.all(np.abs(got.astype(np.float64) - ref) <=
                  _gemm_bound(sub, pk, sc, b, rows.size, n, k, gs, ref))
    D.matmul_int4_grouped(ctx, da, dw, ds, db, None, dy, m, n, k, gs)
    assert np.array_equal(dy.download(), y)


@pytest.mark.parametrize("dtype", [G.GGUF_Q8_0, G.GGUF_Q4_0, G.GGUF_Q4_1])
def test_gguf_blocks(ctx, dtype):
    """Random blocks (every half-precision scale code, NaN / inf included)
    decoded bit for bit; the partial last block reads 0."""
    step = {8: 34, 2: 18, 3: 20}[dtype]
    nb = 4096
    say(f"gguf dtype={dtype} blocks={nb}")
    raw = RNG.integers(0, 256, nb * step).astype(np.uint8)
    h = np.arange(nb, dtype=np.int64) * 16 % 65536             # scale codes across the range
    raw.reshape(nb, step)[:, 0] = h & 255
    raw.reshape(nb, step)[:, 1] = h >> 8
    for n in (nb * 32, nb * 32 - 5, 31, 0):
        got = G.dequant_blocks(raw.tobytes(), 0, n, dtype)
        want = O.dequantize_gguf(raw, n, dtype)
        assert _bits_equal(got, want), (dtype, n)
    n = nb * 32 - 5
    want = O.dequantize_gguf(raw, n, dtype)
    dr = D.DeviceBuffer.from_host(ctx, raw)
    dy = D.DeviceBuffer.empty(ctx, n, np.float32)
    D.dequantize_gguf(ctx, dr, n, dtype, dy)          # four outputs per thread
    assert _bits_equal(dy.download(), want)
    # blocks at an odd address, output not 16-byte aligned: one output per thread
    dr1 = D.DeviceBuffer.from_host(ctx, np.concatenate([np.zeros(1, np.uint8), raw]))
    dy1 = D.DeviceBuffer.empty(ctx, n + 1, np.float32)
    D.dequantize_gguf(ctx, dr1.ptr + 1, n, dtype, dy1.ptr + 4)
    assert _bits_equal(dy1.download()[1:], want)
    for buf in (dr, dy, dr1, dy1):
        buf.close()
    with pytest.raises(ValueError):
        G.dequant_blocks(raw[: step * 3].tobytes(), 0, 4 * 32, dtype)
    with pytest.raises(_lib.TkvHipError):
        G.dequant_blocks(raw.tobytes(), 0, 32, 12)               # Q4_K: the reader's own loop
