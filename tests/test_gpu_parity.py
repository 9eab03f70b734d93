"""GPU parity: libtkv_hip (through its C ABI) against the CPU oracle on the
same seeded inputs.

Bar: bit-exact for codes, scales (f32 bits), INT32 accumulators and the
INT8 dequant epilogue (the IL-derived primary recipe; the north-star
tolerance of 1e-5 relative is therefore met with margin).  FP8 GEMM outputs
are held to the f32-summation bound stated in test_fp8_gemm_*.  Full
GPT-2 sizes are covered through size-independent properties (row / column
checksums of the exact INT32 accumulators and sampled exact outputs).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle as O
from tokenvector.inference_amd import device as D
from tokenvector.inference_amd import quantization as Q
from tokenvector.inference_amd import session as S

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20261201)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _x(n, seed=0, sigma=1.0):
    return O.gi_noise(n, seed, sigma)


def _same_f32(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module")
def ctx(hip):
    c = D.Context(0)
    yield c
    c.close()


# ---------------------------------------------------------------------------
# calibration
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 3, 5, 1000, 1023, 786432])
@pytest.mark.parametrize("sym", [1, 0])
def test_calibrate_minmax(hip, n, sym):
    say(f"calibrate_minmax n={n} sym={sym}")
    x = _x(n, seed=n)
    if n > 100:
        x = O.add_outliers(x, 0.001, 3, 4, 20.0)
    assert Q.calibrate_minmax(x, sym) == O.calibrate_minmax(x, sym)


def test_calibrate_edge_cases(hip):
    say("calibrate edge cases")
    cases = [np.zeros(10, np.float32), np.full(7, 3.0, np.float32),
             np.array([3.0, -0.0, 0.0, 5.0], np.float32), np.array([3.0, 0.0, -0.0], np.float32),
             np.array([-2.0, -0.0, -1.0], np.float32), np.array([1e-12, -1e-12], np.float32)]
    for x in cases:
        for sym in (1, 0):
            g, o = Q.calibrate_minmax(x, sym), O.calibrate_minmax(x, sym)
            assert g.zero_point == o.zero_point
            for a, b in zip(g[:1] + g[2:], o[:1] + o[2:]):
                assert _same_f32(a, b), (x, sym, g, o)
    assert Q.calibrate_minmax([]) == O.quant_identity()


@pytest.mark.parametrize("rows,cols,sym", [(3072, 768, 1), (64, 37, 0), (5, 3072, 1), (17, 1, 0)])
def test_calibrate_per_channel(hip, rows, cols, sym):
    say(f"calibrate_per_channel {rows}x{cols} sym={sym}")
    w = _x(rows * cols, 1, 0.02)
    g = Q.calibrate_per_channel_minmax(w, rows, cols, sym)
    o = O.calibrate_per_channel_minmax(w, rows, cols, sym)
    assert len(g) == rows
    for a, b in zip(g, o):
        assert a.zero_point == b.zero_point
        assert _same_f32([a.scale, a.min_val, a.max_val], [b.scale, b.min_val, b.max_val])
    with pytest.raises(ValueError):
        Q.calibrate_per_channel_minmax(w, rows + 1, cols)


# heavier calibrators (engine.tkv:42-197): equal QuantParams fields.  KL and
# percentile reproduce the reference's arithmetic bit for bit; the MSE search
# sums per-block partials (another order than the reference's loop), so its
# parity is the chosen threshold, exact away from candidates within rounding.
CAL_SIZES = [1, 7, 1000, 65539, 786432, 8192 * 768]


def _same_qp(a, b):
    return a.zero_point == b.zero_point and _same_f32([a.scale, a.min_val, a.max_val],
                                                     [b.scale, b.min_val, b.max_val])


@pytest.mark.parametrize("n", CAL_SIZES)
def test_calibrate_kl(hip, n):
    say(f"calibrate_kl n={n}")
    x = _x(n, 41 + n % 97, 1.0)
    if n > 100:
        x = O.add_outliers(x, 0.001, 3, 4, 20.0)
    for bins, target in [(2048, 128), (512, 32), (64, 8), (4096, 4000), (4096, 4096), (100, 7)]:
        g, o = Q.calibrate_kl(x, bins, target), O.calibrate_kl(x, bins, target)
        assert _same_qp(g, o), (bins, target, g, o)
    z = np.zeros(max(n, 2), np.float32)
    assert _same_qp(Q.calibrate_kl(z), O.calibrate_kl(z))


@pytest.mark.parametrize("bins, target", [(2048, 128), (100, 7), (4096, 16)])
def test_calibrate_kl_bin_edges(hip, bins, target):
    """Elements on the histogram's bin edges: f32(k * bw) and its two f32
    neighbours for every k, where |x| / bw rounds to k or just below it.  The
    kernel's two-sided f32 estimate cannot place these, so every one of them
    takes the f64-division path (per element, inside otherwise fast waves);
    NaN, inf and zeros go the same way.  Compared with the oracle's loop."""
    say(f"calibrate_kl bin edges bins={bins}")
    am = np.float32(3.7)
    bw = float(am) / bins
    k = np.arange(bins + 1, dtype=np.float64)
    e = (k * bw).astype(np.float32)
    x = np.concatenate([e, np.nextafter(e, np.float32(np.inf)), np.nextafter(e, np.float32(0))])
    x = np.minimum(x, am).astype(np.float32)
    rng = np.random.default_rng(bins)
    x = np.concatenate([x, -x, rng.uniform(-3.7, 3.7, 200000).astype(np.float32)])
    rng.shuffle(x)
    x = np.concatenate([x, np.float32([np.nan, 0.0, -0.0])]).astype(np.float32)
    g, o = Q.calibrate_kl(x, bins, target), O.calibrate_kl(x, bins, target)
    assert _same_qp(g, o), (bins, target, g, o)


@pytest.mark.parametrize("n", CAL_SIZES)
def test_calibrate_percentile(hip, n):
    say(f"calibrate_percentile n={n}")
    x = _x(n, 43 + n % 89, 1.0)
    if n > 100:
        x = O.add_outliers(x, 0.001, 3, 4, 20.0)
    x[0] = np.float32(-30.0) if n > 1 else x[0]  # data[0] stays unclipped in the reference
    for pct in (99.99, 50.0, 100.0, 0.5):
        for sym in (1, 0):
            g, o = Q.calibrate_percentile(x, pct, sym), O.calibrate_percentile(x, pct, sym)
            assert _same_qp(g, o), (pct, sym, g, o)
    with pytest.raises(ValueError):
        Q.calibrate_percentile(x, 0.0)


@pytest.mark.parametrize("kind", ["constant", "cluster", "two_values", "ties"])
def test_calibrate_percentile_staging(hip, kind):
    """The second radix pass stages the elements that share the first digit,
    up to 2048 per workgroup, and the third reads only those; a workgroup
    with more sets the spill flag and the third pass reads all of x.  Data
    that overflows the staging everywhere (constant), in some workgroups
    (a dense cluster in one stretch of the tensor), or nowhere (two values,
    exact ties across digits) must all give the oracle's parameters."""
    say(f"calibrate_percentile staging {kind}")
    n = 1 << 22
    rng = np.random.default_rng(11)
    if kind == "constant":
        x = np.full(n, 1.5, np.float32)
    elif kind == "cluster":
        x = rng.standard_normal(n).astype(np.float32)
        x[n // 3: n // 3 + (1 << 20)] = np.float32(0.75) + rng.uniform(0, 1e-6, 1 << 20).astype(
            np.float32)
    elif kind == "two_values":
        x = np.where(rng.uniform(size=n) < 0.5, np.float32(-2.0), np.float32(0.25)).astype(
            np.float32)
    else:
        x = (rng.integers(-1000, 1001, n) / np.float32(64.0)).astype(np.float32)
    for pct in (99.99, 50.0, 3.0):
        for sym in (1, 0):
            g, o = Q.calibrate_percentile(x, pct, sym), O.calibrate_percentile(x, pct, sym)
            assert _same_qp(g, o), (kind, pct, sym, g, o)


@pytest.mark.parametrize("n", [1, 7, 1000, 65539, 786432])
def test_calibrate_mse(hip, n):
    say(f"calibrate_mse n={n}")
    x = _x(n, 47 + n % 83, 1.0)
    if n > 100:
        x = O.add_outliers(x, 0.001, 3, 4, 20.0)
    for nc in (50, 4, 130):
        g, o = Q.calibrate_mse(x, nc), O.calibrate_mse(x, nc)
        assert _same_qp(g, o), (nc, g, o)
    z = np.zeros(max(n, 2), np.float32)
    assert _same_qp(Q.calibrate_mse(z), O.calibrate_mse(z))


@pytest.mark.parametrize("n", [1003, 65539])
def test_calibrators_misaligned_device(ctx, n):
    """The device calibrators on x one float past a 16-byte boundary (the
    scalar load paths), called twice on one context, against the oracle."""
    say(f"calibrators misaligned n={n}")
    x = O.add_outliers(_x(n, 53, 1.0), 0.001, 3, 4, 20.0)
    dx = D.DeviceBuffer.from_host(ctx, np.concatenate([np.zeros(1, np.float32), x]))
    p = D.params_buffer(ctx)
    xp = dx.ptr + 4
    for _ in range(2):
        D.calibrate_kl(ctx, xp, n, p, 512, 32)
        g = D.read_params(p)
        assert _same_qp(g, O.calibrate_kl(x, 512, 32))
        D.calibrate_percentile(ctx, xp, n, p, 99.9, 0)
        assert _same_qp(D.read_params(p), O.calibrate_percentile(x, 99.9, 0))
        D.calibrate_mse(ctx, xp, n, p, 37)
        assert _same_qp(D.read_params(p), O.calibrate_mse(x, 37))


def _same_f32_nan(a, b):
    """Bit-exact, except that any NaN matches any NaN: the sign and payload of
    a NaN made by arithmetic differ between x86 and the GPU and carry no
    meaning in the reference."""
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    na, nb = np.isnan(a), np.isnan(b)
    return (a.shape == b.shape and np.array_equal(na, nb)
            and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


def _same_qp_nan(a, b):
    return a.zero_point == b.zero_point and _same_f32_nan([a.scale, a.min_val, a.max_val],
                                                         [b.scale, b.min_val, b.max_val])


def _nan_cases(n):
    """NaN first (calibrate_minmax and DynamicQuantizeLinear seed min / max
    with x[0], so the result is NaN), NaN inside (skipped by every strict
    comparison), all NaN (the absmax loops that start from 0 give 0), a
    finite first element before NaN only, and +inf first."""
    base = _x(n, 71 + n % 13, 1.0)
    first = base.copy(); first[0] = np.nan
    inside = base.copy(); inside[n // 2] = np.nan; inside[n - 1] = np.nan
    fin = np.full(n, np.nan, np.float32); fin[0] = -0.75
    inf = base.copy(); inf[0] = np.inf; inf[n // 3] = np.nan
    return {"first": first, "inside": inside, "all": np.full(n, np.nan, np.float32),
            "finite-first": fin, "inf-first": inf}


@pytest.mark.parametrize("n", [2, 1000, 65539, 786432])
def test_nan_inputs_tensor(ctx, n):
    """NaN handling of the per-tensor calibrators and the fused calibrate +
    quantize, against the oracle (engine.tkv:13-36, 165-197, 216-226;
    session.tkv:2853-2876).  calibrate_kl and calibrate_percentile are left
    out: the reference's histogram index and heap sort of a NaN are undefined
    (int(NaN) as a list index, comparisons that are always false)."""
    say(f"NaN inputs, tensor n={n}")
    dq = D.DeviceBuffer.empty(ctx, n, np.int8)
    p = D.params_buffer(ctx)
    dyn = S.new_node("dyn", S.OperatorType_DynamicQuantizeLinear)
    for name, x in _nan_cases(n).items():
        for sym in (1, 0):
            g, o = Q.calibrate_minmax(x, sym), O.calibrate_minmax(x, sym)
            assert _same_qp_nan(g, o), (name, sym, g, o)
        g, o = Q.calibrate_mse(x, 20), O.calibrate_mse(x, 20)
        assert _same_qp_nan(g, o), (name, "mse", g, o)
        dx = D.DeviceBuffer.from_host(ctx, x)
        D.quantize_int8_dynamic_tensor(ctx, dx.ptr, n, dq, p)
        want = O.calibrate_minmax(x, 1)
        got = D.read_params(p)
        assert _same_f32_nan([got.scale, got.min_val, got.max_val],
                             [want.scale, want.min_val, want.max_val]), (name, got, want)
        assert np.array_equal(dq.download().astype(np.int32),
                              O.quantize_int8_symmetric(x, want.scale)), name
        if n <= 65539:
            yq, ys, yz = dyn.execute([(x, [n])], [])
            oq, oys, oyz = O.dynamic_quantize_linear(x)
            assert np.array_equal(yq, oq) and _same_f32_nan([ys, yz], [oys, oyz]), name


@pytest.mark.parametrize("cols", [768, 700, 3072, 37, 4])
def test_nan_inputs_rows(hip, cols):
    """Per-row NaN handling: calibrate_per_channel_minmax seeds each row's
    min / max with its first element (engine.tkv:202-213 -> 13-36);
    quantize_dynamic_int8_rowwise takes max |x| from 0 (engine.tkv:266-285),
    so a row of NaN gets the 1e-8 floor.  Row widths cover the register-held
    row kernel with whole and partial float4 lanes (768, 700, 3072) and the
    scalar row kernel (37)."""
    say(f"NaN inputs, rows cols={cols}")
    rows = 24
    x = _x(rows * cols, 91 + cols, 1.0).reshape(rows, cols)
    x[1, 0] = np.nan                    # NaN first
    x[2, cols // 2] = np.nan            # NaN inside
    x[3, :] = np.nan                    # all NaN
    x[4, 1:] = np.nan                   # finite first, then NaN only
    x[5, 0] = np.inf                    # +inf first
    x[6, cols - 1] = -np.inf            # -inf last
    x[7, :] = 0.0                       # all zero: 1e-8 floor
    x = x.reshape(-1)
    for sym in (1, 0):
        g = Q.calibrate_per_channel_minmax(x, rows, cols, sym)
        o = O.calibrate_per_channel_minmax(x, rows, cols, sym)
        assert all(_same_qp_nan(a, b) for a, b in zip(g, o)), sym
    q = np.zeros(rows * cols, np.int32)
    so = np.zeros(rows, np.float32)
    Q.quantize_dynamic_int8_rowwise(x, q, rows, cols, so)
    oq, os_ = O.quantize_dynamic_int8_rowwise(x, rows, cols)
    assert np.array_equal(q, oq) and _same_f32_nan(so, os_)


@pytest.mark.parametrize("rows,cols", [(3 * 8192 + 5, 768), (2 * 8192 + 3, 700), (20000, 256)])
def test_dynamic_rowwise_many_rows(ctx, rows, cols):
    """More rows than the row kernel's resident waves (8 blocks of 4 waves
    per CU), so each wave walks several rows through both register sets and
    the prefetch past the last row; int8 codes through the device entry point
    and int32 codes through the host mirror, against the oracle."""
    say(f"dynamic rowwise many rows {rows}x{cols}")
    x = _x(rows * cols, 13 + cols, 1.0)
    x[cols * 7: cols * 8] = 0.0
    oq, os_ = O.quantize_dynamic_int8_rowwise(x, rows, cols)
    dx = D.DeviceBuffer.from_host(ctx, x)
    dq = D.DeviceBuffer.empty(ctx, rows * cols, np.int8)
    ds = D.DeviceBuffer.empty(ctx, rows, np.float32)
    D.quantize_dynamic_int8_rowwise(ctx, dx, rows, cols, dq, ds)
    assert np.array_equal(dq.download().astype(np.int32), oq)
    assert _same_f32(ds.download(), os_)
    q = np.zeros(rows * cols, np.int32)
    so = np.zeros(rows, np.float32)
    Q.quantize_dynamic_int8_rowwise(x, q, rows, cols, so)
    assert np.array_equal(q, oq) and _same_f32(so, os_)


# ---------------------------------------------------------------------------
# quantize / dequantize (config 2 shapes)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m", [1024, 8192, 65536])
def test_config2_quantize_int8_and_fp8(hip, m):
    say(f"config2 quantize M={m}")
    x = O.add_outliers(_x(m * 768, 0, 1.0), 0.001, 3, 4, 20.0)
    p = Q.calibrate_minmax(x, 1)
    assert p == O.calibrate_minmax(x, 1)
    for recipe in (Q.PRIMARY, Q.ALTERNATE):
        q = np.zeros(x.size, np.int32)
        Q.quantize_int8_symmetric(x, q, p.scale, recipe)
        assert np.array_equal(q, O.quantize_int8_symmetric(x, p.scale, recipe))
    qr = np.zeros(x.size, np.int32)
    so = np.zeros(m, np.float32)
    Q.quantize_dynamic_int8_rowwise(x, qr, m, 768, so)
    oq, os_ = O.quantize_dynamic_int8_rowwise(x, m, 768)
    assert np.array_equal(qr, oq) and _same_f32(so, os_)
    qf = np.zeros(x.size, np.int32)
    Q.quantize_fp8_e4m3(x, qf)
    assert np.array_equal(qf, O.quantize_fp8_e4m3(x))
    rows = Q.calibrate_per_channel_minmax(x, m, 768, 1)
    assert _same_f32([r.scale for r in rows], [r.scale for r in O.calibrate_per_channel_minmax(x, m, 768, 1)])


def test_quantize_int8_edges(hip):
    say("quantize edges")
    k = np.arange(-300, 300)
    ties = ((k + 0.5) / 16.0).astype(np.float32)
    special = np.array([1e30, -1e30, np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-45, -1e-45], np.float32)
    for x, scale in [(ties, 2.0 ** -4), (special, 0.5), (_x(1001, 9), 0.013), (_x(7, 2), 1e-9),
                     (_x(33, 4), 0.0)]:
        for recipe in (Q.PRIMARY, Q.ALTERNATE):
            q = np.zeros(x.size, np.int32)
            Q.quantize_int8_symmetric(x, q, scale, recipe)
            assert np.array_equal(q, O.quantize_int8_symmetric(x, scale, recipe)), (scale, recipe)
    with pytest.raises(ValueError):
        Q.quantize_int8_symmetric(ties, np.zeros(3, np.int32), 0.1)


@pytest.mark.parametrize("rows,cols", [(3072, 768), (768, 3072), (9, 37), (4, 1)])
def test_quantize_per_channel_and_dequantize(hip, rows, cols):
    say(f"per-channel {rows}x{cols}")
    w = _x(rows * cols, 1, 0.02)
    sc = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, rows, cols)], np.float32)
    sc[0] = 0.0  # floor to 1e-8
    q = np.zeros(rows * cols, np.int32)
    Q.quantize_int8_per_channel(w, q, rows, cols, sc)
    oq = O.quantize_int8_per_channel(w, rows, cols, sc)
    assert np.array_equal(q, oq)
    d = np.zeros(rows * cols, np.float32)
    Q.dequantize_int8_per_channel(oq, d, rows, cols, sc)
    assert _same_f32(d, O.dequantize_int8_per_channel(oq, rows, cols, sc))
    d2 = np.zeros(rows * cols, np.float32)
    Q.dequantize_int8_symmetric(oq, d2, np.float32(0.0173))
    assert _same_f32(d2, O.dequantize_int8_symmetric(oq, np.float32(0.0173)))
    with pytest.raises(ValueError):
        Q.quantize_int8_per_channel(w, q, rows, cols, sc[:-1] if rows > 1 else [])


@pytest.mark.parametrize("rows,cols", [(1, 768), (32, 3072), (5, 37), (3, 4), (9000, 3072),
                                       (3000, 1536)])
def test_dynamic_rowwise_shapes(hip, rows, cols):
    say(f"dynamic rowwise {rows}x{cols}")
    x = _x(rows * cols, 5, 1.0)
    x[:cols] = 0.0  # an all-zero row floors to 1e-8
    q = np.zeros(rows * cols, np.int32)
    so = np.zeros(rows, np.float32)
    Q.quantize_dynamic_int8_rowwise(x, q, rows, cols, so)
    oq, os_ = O.quantize_dynamic_int8_rowwise(x, rows, cols)
    assert np.array_equal(q, oq) and _same_f32(so, os_)


# ---------------------------------------------------------------------------
# FP8 e4m3 codec
# ---------------------------------------------------------------------------

def test_fp8_encode_bit_patterns(ctx):
    """Every f32 bit pattern with biased exponent 96..160 (both signs; all
    encode decisions of e4m3 happen there) plus 2^24 random patterns."""
    chunk = 1 << 26
    xb = D.DeviceBuffer.empty(ctx, chunk, np.float32)
    qb = D.DeviceBuffer.empty(ctx, chunk, np.uint8)
    starts = []
    for sign in (0, 1):
        lo = (sign << 31) | (96 << 23)
        hi = (sign << 31) | (161 << 23)
        starts += list(range(lo, hi, chunk))
    for s in starts:
        bits = np.arange(s, s + chunk, dtype=np.uint64).astype(np.uint32)
        xb.upload(bits.view(np.float32))
        D.quantize_fp8_e4m3(ctx, xb, chunk, qb)
        got = qb.download()
        want = O.fp8_encode_bits(bits)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, hex(int(bits[bad[0]]))
    say(f"fp8 encode: {len(starts)} chunks of 2^26 patterns")
    bits = RNG.integers(0, 2 ** 32, chunk, dtype=np.uint64).astype(np.uint32)
    xb.upload(bits.view(np.float32))
    D.quantize_fp8_e4m3(ctx, xb, chunk, qb)
    assert np.array_equal(qb.download(), O.fp8_encode_bits(bits))


# Per-tensor sizes: tiny and ragged (n % 4 tails), one float4 per thread of a
# 256 x 512 grid and just past it, the GPT-2 activation sizes, and one past
# the largest; every call runs calibrate + quantize back to back.
GRID_CHUNK = 256 * 512 * 4
DYN_SIZES = [1, 3, 4, 1000, 1023, GRID_CHUNK, GRID_CHUNK + 1, 5 * GRID_CHUNK + 7,
             8192 * 768, 8192 * 3072, 8192 * 3072 + 4]


@pytest.mark.parametrize("n,offset", [(n, 0) for n in DYN_SIZES] + [(1000, 1), (8192 * 768, 1)])
def test_int8_dynamic_tensor(ctx, n, offset):
    """calibrate_minmax(x, 1) + quantize_int8_symmetric on the device in one
    call (engine.tkv:13-36, 216-226): QuantParams and codes bit-exact, for
    every size aligned and for two sizes with x one float off 16 bytes."""
    say(f"int8 dynamic tensor n={n} offset={offset}")
    x = _x(n, 17 + n % 1000, 1.0)
    if n > 100:
        x = O.add_outliers(x, 0.001, 3, 4, 20.0)
    dx = D.DeviceBuffer.from_host(ctx, np.concatenate([np.zeros(offset, np.float32), x]))
    dq = D.DeviceBuffer.empty(ctx, n, np.int8)
    p = D.params_buffer(ctx)
    for _ in range(2):  # twice: the second call reuses the context's partials
        D.quantize_int8_dynamic_tensor(ctx, dx.ptr + 4 * offset, n, dq, p)
        want_p = O.calibrate_minmax(x, 1)
        got_p = D.read_params(p)
        assert _same_f32([got_p.scale, got_p.min_val, got_p.max_val],
                         [want_p.scale, want_p.min_val, want_p.max_val])
        assert np.array_equal(dq.download().astype(np.int32),
                              O.quantize_int8_symmetric(x, want_p.scale))


# Activation-sized tensors around 8192 x 768 and beyond (float4 tails of 0 and
# 4 elements past multiples of 256 * 512 * 4).  From 16 Mi elements on, the
# single-pass kernel runs (one 768-thread workgroup per CU holding 32 float4
# per thread on chip: 8192 x 3072 exactly fills 256 CUs, and 4 elements more
# take the two-kernel path).
RES_UNIT = 256 * 512 * 4
RES_SIZES = [RES_UNIT * r + d for r in (4, 8, 16, 24, 32) for d in (0, 4)] + [2 ** 20] + \
    [8192 * 3072, 8192 * 3072 + 4, 2 ** 24 + 12]


def _res_input(n, seed):
    x = _x(n, seed, 1.0)
    return O.add_outliers(x, 0.001, 3, 4, 20.0)


def _dyn_quant(ctx, x, two_pass=False, spin=-1):
    n = x.size
    dx = D.DeviceBuffer.from_host(ctx, x)
    dq = D.DeviceBuffer.empty(ctx, n, np.int8)
    p = D.params_buffer(ctx)
    ctx.set_tuning(D.TUNE_QUANT_TWO_PASS, 1 if two_pass else -1)
    ctx.set_tuning(D.TUNE_GRID_SPIN, spin)
    try:
        D.quantize_int8_dynamic_tensor(ctx, dx, n, dq, p)
        ctx.synchronize()
    finally:
        ctx.set_tuning(D.TUNE_QUANT_TWO_PASS, -1)
        ctx.set_tuning(D.TUNE_GRID_SPIN, -1)
    return D.read_params(p), dq.download().astype(np.int32)


@pytest.mark.parametrize("n", RES_SIZES)
def test_int8_dynamic_tensor_activation_sizes(ctx, n):
    """calibrate + quantize on activation-sized tensors: QuantParams and codes
    bit-exact against the oracle."""
    say(f"int8 dynamic tensor activation size n={n}")
    x = _res_input(n, 5 + n % 997)
    got_p, got_q = _dyn_quant(ctx, x)
    want_p = O.calibrate_minmax(x, 1)
    assert _same_f32([got_p.scale, got_p.min_val, got_p.max_val],
                     [want_p.scale, want_p.min_val, want_p.max_val])
    assert np.array_equal(got_q, O.quantize_int8_symmetric(x, want_p.scale))


@pytest.mark.parametrize("case", ["nan_first", "nan_inside", "inf", "zeros", "tiny", "ties",
                                  "negative_extreme"])
@pytest.mark.parametrize("n", [3 * RES_UNIT, 33 * RES_UNIT])
def test_int8_dynamic_tensor_specials(ctx, case, n):
    """NaN (first element and inside), infinities, an all-zero tensor (the
    1e-8 scale floor), values below the floor, exact .5 ties of x * inv and a
    negative extreme, at an activation size for each path (two kernels, single
    pass): bit-exact against the oracle, and the single-pass size also equal
    to the two-kernel path's result."""
    say(f"int8 dynamic tensor special={case} n={n}")
    x = _res_input(n, 77)
    if case == "nan_first":
        x[0] = np.nan
    elif case == "nan_inside":
        x[RNG.integers(1, n, 64)] = np.nan
    elif case == "inf":
        x[12345] = np.inf
        x[n - 1] = -np.inf
    elif case == "zeros":
        x[:] = 0.0
        x[7] = -0.0
    elif case == "tiny":
        x = (x * np.float32(1e-12)).astype(np.float32)
    elif case == "ties":
        # amax 127 gives scale 1 and inv 1: every k + 0.5 is an exact tie
        x = (np.round(x * 20) / 2).astype(np.float32)
        x[0] = 127.0
        x = np.clip(x, -127.0, 127.0).astype(np.float32)
    elif case == "negative_extreme":
        x[999] = -50.0
    got_p, got_q = _dyn_quant(ctx, x)
    want_p = O.calibrate_minmax(x, 1)
    assert _same_f32([got_p.scale, got_p.min_val, got_p.max_val],
                     [want_p.scale, want_p.min_val, want_p.max_val])
    want_q = O.quantize_int8_symmetric(x, want_p.scale)
    assert np.array_equal(got_q, want_q)
    if n >= 2 ** 24:
        two_p, two_q = _dyn_quant(ctx, x, two_pass=True)
        assert _same_f32([two_p.scale, two_p.min_val, two_p.max_val],
                         [got_p.scale, got_p.min_val, got_p.max_val])
        assert np.array_equal(two_q, want_q)


@pytest.mark.parametrize("spin", [0, 1])
def test_int8_dynamic_tensor_barrier_give_up(ctx, spin):
    """The single-pass kernel's bounded grid barrier with the spin limit set
    from the host to 0 or 1 poll: every workgroup (or all but the leader's
    gather) gives up and scans the whole tensor itself.  QuantParams and codes
    bit-exact against the oracle at 8192 x 3072 (with a NaN first element too),
    and an ordinary call right after, whose barrier must still see consistent
    slot generations."""
    n = 8192 * 3072
    for case in ("plain", "nan_first"):
        say(f"int8 dynamic tensor give-up spin={spin} {case} n={n}")
        x = _res_input(n, 91)
        if case == "nan_first":
            x[0] = np.nan
        got_p, got_q = _dyn_quant(ctx, x, spin=spin)
        want_p = O.calibrate_minmax(x, 1)
        assert _same_f32([got_p.scale, got_p.min_val, got_p.max_val],
                         [want_p.scale, want_p.min_val, want_p.max_val]), (spin, case)
        want_q = O.quantize_int8_symmetric(x, want_p.scale)
        assert np.array_equal(got_q, want_q), (spin, case)
        again_p, again_q = _dyn_quant(ctx, x)
        assert _same_f32([again_p.scale], [want_p.scale]) and np.array_equal(again_q, want_q)


def test_int8_dynamic_tensor_repeated(ctx):
    """Back-to-back calls of different sizes on one context, no sync between
    them (the context's partials are reused by every call)."""
    sizes = [RES_SIZES[0], 8192 * 3072, RES_SIZES[5], 2 ** 20, 2 ** 24 + 12, RES_SIZES[2]] * 2
    xs = {n: _res_input(n, n % 101) for n in set(sizes)}
    bufs = {n: (D.DeviceBuffer.from_host(ctx, xs[n]), D.DeviceBuffer.empty(ctx, n, np.int8))
            for n in xs}
    ps = [D.params_buffer(ctx) for _ in sizes]
    for i, n in enumerate(sizes):
        D.quantize_int8_dynamic_tensor(ctx, bufs[n][0], n, bufs[n][1], ps[i])
    ctx.synchronize()
    for i, n in enumerate(sizes):
        want_p = O.calibrate_minmax(xs[n], 1)
        assert _same_f32([D.read_params(ps[i]).scale], [want_p.scale])
    for n in xs:
        want_p = O.calibrate_minmax(xs[n], 1)
        assert np.array_equal(bufs[n][1].download().astype(np.int32),
                              O.quantize_int8_symmetric(xs[n], want_p.scale))


@pytest.mark.parametrize("n", [1, 1000, 5 * GRID_CHUNK + 7, 8192 * 768, 32 * GRID_CHUNK,
                               8192 * 3072])
def test_fp8_dynamic_tensor(ctx, n):
    """Per-tensor FP8 activation quantize (extension used by the FP8 linear):
    scale = fl32(max|x| / 240), codes = encode(fl32(x * fl32(1 / scale)))."""
    say(f"fp8 dynamic tensor n={n}")
    x = _x(n, 31, 1.0)
    if n > 100:
        x = O.add_outliers(x, 0.001, 3, 4, 20.0)
    dx = D.DeviceBuffer.from_host(ctx, x)
    dq = D.DeviceBuffer.empty(ctx, n, np.uint8)
    p = D.params_buffer(ctx)
    D.quantize_fp8_e4m3_dynamic_tensor(ctx, dx, n, dq, p)
    am = max(float(np.max(np.abs(x.astype(np.float64)))), 1e-8)
    scale = np.float32(am / 240.0)
    assert _same_f32([D.read_params(p).scale], [scale])
    inv = np.float32(1.0) / scale
    want = O.fp8_encode_bits((x * inv).astype(np.float32).view(np.uint32))
    assert np.array_equal(dq.download(), want)


def test_fp8_decode_all_codes(hip):
    say("fp8 decode")
    codes = np.arange(-128, 128, dtype=np.int32)
    d = np.zeros(256, np.float32)
    Q.dequantize_fp8_e4m3(codes, d)
    assert _same_f32(d, O.dequantize_fp8_e4m3(codes))


# ---------------------------------------------------------------------------
# INT8 GEMM
# ---------------------------------------------------------------------------

SHAPES_SMALL = [(1, 1, 1), (3, 5, 17), (37, 100, 96), (130, 200, 768), (64, 64, 3072), (257, 129, 200)]


@pytest.mark.parametrize("m,n,k", SHAPES_SMALL)
def test_int8_accumulators(hip, m, n, k):
    say(f"int8 accum {m}x{n}x{k}")
    a = RNG.integers(-128, 128, (m, k)).astype(np.int32)
    w = RNG.integers(-128, 128, (n, k)).astype(np.int32)
    acc = Q.matmul_int8_accum(a, w, m, n, k).reshape(m, n)
    assert np.array_equal(acc, a.astype(np.int64) @ w.astype(np.int64).T)


@pytest.mark.parametrize("m,n,k", SHAPES_SMALL[1:])
@pytest.mark.parametrize("recipe", [Q.PRIMARY, Q.ALTERNATE])
def test_int8_gemm_epilogues(hip, m, n, k, recipe):
    say(f"int8 gemm {m}x{n}x{k} recipe={recipe}")
    a = RNG.integers(-127, 128, (m, k)).astype(np.int32)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int32)
    sa = np.float32(0.0213)
    sw = RNG.uniform(1e-4, 3e-4, n).astype(np.float32)
    b = RNG.normal(0, 0.01, n).astype(np.float32)
    for bias in (b, None):
        y = np.zeros(m * n, np.float32)
        Q.matmul_int8_recipe(a, w, bias, y, m, n, k, sa, 0.0, sw, recipe)
        assert _same_f32(y, O.matmul_int8_per_channel(a, w, bias, m, n, k, sa, sw, recipe))
        y = np.zeros(m * n, np.float32)
        Q.matmul_int8_recipe(a, w, bias, y, m, n, k, sa, np.float32(3.1e-4), None, recipe)
        assert _same_f32(y, O.matmul_int8_symmetric(a, w, bias, m, n, k, sa, np.float32(3.1e-4), recipe))


def _c1_inputs():
    x = _x(1024 * 768, 0, 1.0)
    w = _x(3072 * 768, 1, 0.02)
    b = _x(3072, 2, 0.01)
    return x, w, b


def test_config1_pipeline_bit_exact(hip):
    """Config 1: X [1024,768] per-tensor, W [3072,768] per-channel, INT8
    GEMM, dequant + bias -- host mirrors end to end vs the oracle."""
    say("config1 pipeline")
    x, w, b = _c1_inputs()
    m, n, k = 1024, 3072, 768
    pw = Q.calibrate_per_channel_minmax(w, n, k)
    sw = np.array([p.scale for p in pw], np.float32)
    wq = np.zeros(n * k, np.int32)
    Q.quantize_int8_per_channel(w, wq, n, k, sw)
    px = Q.calibrate_minmax(x, 1)
    xq = np.zeros(m * k, np.int32)
    Q.quantize_int8_symmetric(x, xq, px.scale)
    y = np.zeros(m * n, np.float32)
    Q.matmul_int8_per_channel(xq, wq, b, y, m, n, k, px.scale, sw)
    # oracle chain
    osw = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, n, k)], np.float32)
    owq = O.quantize_int8_per_channel(w, n, k, osw)
    opx = O.calibrate_minmax(x, 1)
    oxq = O.quantize_int8_symmetric(x, opx.scale)
    assert _same_f32(sw, osw) and np.array_equal(wq, owq)
    assert px == opx and np.array_equal(xq, oxq)
    oy = O.matmul_int8_per_channel(oxq, owq, b, m, n, k, opx.scale, osw, threads=O.host_threads())
    assert _same_f32(y, oy)
    # session mirror of the QuantizedGemm node gives the same bits
    node = S.new_node("qg", S.OperatorType_QuantizedGemm)
    node.scale_a = px.scale
    node.scales_w = list(sw)
    (y2,) = node.execute([(xq, [m, k]), (wq, [n, k]), (b, [n])], [[m, n]])
    assert _same_f32(y2, oy)


GPT2 = [(2304, 768), (768, 768), (3072, 768), (768, 3072)]


@pytest.mark.parametrize("n,k", GPT2)
def test_int8_full_size_properties(ctx, n, k):
    """Config 3 shapes (M = 8192): exact INT32 row / column checksums and
    4096 sampled accumulators; the dequant epilogue checked on those samples."""
    m = 8192
    say(f"int8 full-size {m}x{n}x{k}")
    a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    da, dw = D.DeviceBuffer.from_host(ctx, a), D.DeviceBuffer.from_host(ctx, w)
    dacc = D.DeviceBuffer.empty(ctx, (m, n), np.int32)
    D.matmul_int8_accum(ctx, da, dw, m, n, k, dacc)
    acc = dacc.download().astype(np.int64)
    a64, w64 = a.astype(np.int64), w.astype(np.int64)
    assert np.array_equal(acc.sum(axis=0), a64.sum(axis=0) @ w64.T)
    assert np.array_equal(acc.sum(axis=1), a64 @ w64.sum(axis=0))
    ii, jj = RNG.integers(0, m, 4096), RNG.integers(0, n, 4096)
    assert np.array_equal(acc[ii, jj], np.einsum("ik,ik->i", a64[ii], w64[jj]))
    # fused epilogue on the same launch shape
    sa = np.array([0.0213], np.float32)
    sw = RNG.uniform(1e-4, 3e-4, n).astype(np.float32)
    b = RNG.normal(0, 0.01, n).astype(np.float32)
    dsa, dsw, db = (D.DeviceBuffer.from_host(ctx, v) for v in (sa, sw, b))
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    D.matmul_int8(ctx, da, dw, m, n, k, dsa, 0, 0.0, dsw, db, dy)
    y = dy.download()
    want = ((acc[ii, jj].astype(np.float64) * np.float64(sa[0])) * sw[jj].astype(np.float64)
            + b[jj].astype(np.float64)).astype(np.float32)
    assert _same_f32(y[ii, jj], want)


@pytest.mark.parametrize("nbytes", [16, 4096, 1000003, 48 << 20])
def test_memcpy_d2d(ctx, nbytes):
    say(f"memcpy_d2d {nbytes}")
    src = RNG.integers(0, 256, nbytes, dtype=np.uint8)
    ds = D.DeviceBuffer.from_host(ctx, src)
    dd = D.DeviceBuffer.empty(ctx, nbytes, np.uint8)
    dd.copy_from(ds)
    assert np.array_equal(dd.download(), src)


def test_matmul_integer_node(hip):
    say("MatMulInteger")
    node = S.new_node("mi", S.OperatorType_MatMulInteger)
    (y,) = node.execute([([1, 2, 3, 4], [2, 2]), ([1, 1, 1, 1], [2, 2])], [[2, 2]])
    assert list(y) == [3, 3, 7, 7]        # inference_tests.tkv:896-922
    m, n, k = 33, 17, 45
    a = RNG.integers(-128, 128, m * k - 5).astype(np.int32)
    b = RNG.integers(-128, 128, k * n).astype(np.int32)
    (y,) = node.execute([(a, [m, k]), (b, [k, n])], [[m * n - 2]])
    assert np.array_equal(y, O.matmul_integer(a, b, m * n - 2, m, n, k))


def test_qlinear_matmul_node(hip):
    """QLinearMatMul node mirror (session.tkv:1992-2071) against the oracle,
    bit-exact: the ONNX-style 2x2 case, random zero points and scales at tile
    edges, short A / B / Y, sy == 0, K == 0, both recipes."""
    say("QLinearMatMul node")
    node = S.new_node("ql", S.OperatorType_QLinearMatMul)
    one = lambda v: (np.array([v], np.float32), [1])
    (y,) = node.execute([([1, 2, 3, 4], [2, 2]), one(0.5), one(0), ([1, 1, 1, 1], [2, 2]),
                         one(0.5), one(0), one(0.25), one(0)], [[2, 2]])
    assert list(y) == [3, 3, 7, 7]
    cases = [(1, 1, 1), (2, 3, 5), (33, 17, 45), (129, 200, 300), (300, 500, 384), (5, 7, 0)]
    for ci, (m, n, k) in enumerate(cases):
        a = RNG.integers(-128, 128, m * k).astype(np.int32)
        b = RNG.integers(-128, 128, k * n).astype(np.int32)
        if ci == 2:
            a, b = a[:-5], b[:-7]
        zpa, zpw, zpy = (int(v) for v in RNG.integers(-30, 31, 3))
        sa, sw = (float(np.float32(v)) for v in RNG.uniform(0.001, 0.05, 2))
        if ci == 1:
            sy = 0.0
        else:  # map the sums' range onto about +-100 codes
            av = np.zeros(m * k, np.int64)
            av[:a.size] = a.astype(np.int64) - zpa
            bv = np.zeros(k * n, np.int64)
            bv[:b.size] = b.astype(np.int64) - zpw
            span = max(1, int(np.abs(av.reshape(m, k) @ bv.reshape(k, n)).max())) if k else 1
            sy = float(np.float32(sa * sw * span / 100.0))
        ny = m * n - (3 if ci == 3 else 0)
        for recipe in (0, 1):
            (y,) = [node._qlinear_matmul([(a, [m, k]), one(sa), one(zpa), (b, [k, n]), one(sw),
                                          one(zpw), one(sy), one(zpy)], [ny], recipe)]
            want = O.qlinear_matmul(a, sa, zpa, b, sw, zpw, sy, zpy, ny, m, n, k, recipe)
            assert np.array_equal(y, want), (m, n, k, recipe)
            if ci >= 3 and k > 0:
                assert np.unique(y).size > 50, "requantized codes should spread over the range"
    # zero points too large for the int32 fast path (exact f64 correction), and
    # an f32-chain multiplier that overflows to inf (alternate recipe)
    m, n, k = 40, 70, 300
    a = RNG.integers(-128, 128, m * k).astype(np.int32)
    b = RNG.integers(-128, 128, k * n).astype(np.int32)
    for (sa, zpa, sw, zpw, sy, zpy) in [(0.01, 20000, 0.02, -15000, 2.0e6, 3),
                                         (1e30, 2, 1e30, -1, 1.0, -5)]:
        for recipe in (0, 1):
            (y,) = [node._qlinear_matmul([(a, [m, k]), one(sa), one(zpa), (b, [k, n]), one(sw),
                                          one(zpw), one(sy), one(zpy)], [m * n], recipe)]
            want = O.qlinear_matmul(a, sa, zpa, b, sw, zpw, sy, zpy, m * n, m, n, k, recipe)
            assert np.array_equal(y, want), (zpa, zpw, sa, recipe)


def test_qdq_nodes(hip):
    say("Q/DQ nodes")
    x = _x(2 * 3 * 40, 8, 3.0).reshape(2, 3, 40)
    q = S.new_node("q", S.OperatorType_QuantizeLinear)
    (y,) = q.execute([(x, [2, 3, 40]), (np.array([0.05], np.float32), [1]),
                      (np.array([3.0], np.float32), [1])], [[2, 3, 40]])
    assert np.array_equal(y, O.quantize_linear(x, [0.05], 3))
    sc = np.array([0.02, 0.1, 1e-13], np.float32)
    (y,) = q.execute([(x, [2, 3, 40]), (sc, [3])], [[2, 3, 40]])
    assert np.array_equal(y, O.quantize_linear(x, sc, 0, 2, 3, 40))
    dq = S.new_node("dq", S.OperatorType_DequantizeLinear)
    (d,) = dq.execute([(y, [2, 3, 40]), (sc, [3])], [[2, 3, 40]])
    assert _same_f32(d, O.dequantize_linear(y, sc, 0, 2, 3, 40))
    dyn = S.new_node("dyn", S.OperatorType_DynamicQuantizeLinear)
    for v in ([0.0, 1.0, 2.0], x.reshape(-1), np.full(5, 2.5, np.float32), -np.abs(x.reshape(-1))):
        yq, ys, yz = dyn.execute([(np.asarray(v, np.float32), [len(v)])], [])
        oq, oys, oyz = O.dynamic_quantize_linear(v)
        assert np.array_equal(yq, oq) and _same_f32(ys, [oys]) and _same_f32(yz, [oyz])


# ---------------------------------------------------------------------------
# FP8 GEMM (f32 accumulation: bound, not bits)
# ---------------------------------------------------------------------------

def _fp8_codes(shape, allow_subnormal):
    codes = [c for c in range(256) if (c & 0x7F) != 0x7F and
             (allow_subnormal or ((c >> 3) & 15) != 0 or (c & 7) == 0)]
    return (RNG.choice(codes, shape) - 128).astype(np.int32)


def _fp8_ref(a, w, bias, m, n, k):
    """Reference output, sum_k |a_k w_k| and the ulp of the reference output."""
    _, asum = O.matmul_fp8_e4m3_exact(a, w, m, n, k)
    ref = O.matmul_fp8_e4m3(a, w, bias, m, n, k)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return ref.astype(np.float64), asum, ulp


FP8_SHAPES = [(1, 1, 64), (37, 100, 96), (128, 256, 768), (64, 96, 3072), (130, 200, 200)]


@pytest.mark.parametrize("m,n,k", FP8_SHAPES)
def test_fp8_gemm_reference_products(hip, m, n, k):
    """matmul_fp8_e4m3 drop-in: the reference decoder's products (subnormal
    codes included) summed at f32-class precision.  Stated bound:
    |y - y_ref| <= 8 * 2^-24 * sum_k |a_k w_k| + ulp(y_ref)."""
    say(f"fp8 gemm (reference products) {m}x{n}x{k}")
    a, w = _fp8_codes((m, k), True), _fp8_codes((n, k), True)
    b = RNG.normal(0, 1, n).astype(np.float32)
    y = np.zeros(m * n, np.float32)
    Q.matmul_fp8_e4m3(a, w, b, y, m, n, k)
    ref, asum, ulp = _fp8_ref(a, w, b, m, n, k)
    err = np.abs(y.astype(np.float64) - ref)
    tol = 8 * 2.0 ** -24 * asum + ulp
    assert np.all(err <= tol), float((err / tol).max())


@pytest.mark.parametrize("m,n,k", FP8_SHAPES)
def test_fp8_gemm_fast(ctx, m, n, k):
    """Full-rate FP8 MFMA path, normal codes: stated bound
    |y - y_ref| <= 2^-10 * sum_k |a_k w_k| + ulp(y_ref)."""
    say(f"fp8 gemm (fast) {m}x{n}x{k}")
    a, w = _fp8_codes((m, k), False), _fp8_codes((n, k), False)
    b = RNG.normal(0, 1, n).astype(np.float32)
    da = D.DeviceBuffer.from_host(ctx, (a + 128).astype(np.uint8))
    dw = D.DeviceBuffer.from_host(ctx, (w + 128).astype(np.uint8))
    db = D.DeviceBuffer.from_host(ctx, b)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    D.matmul_fp8_e4m3(ctx, da, dw, m, n, k, None, 0, None, db, dy, fast=True)
    ref, asum, ulp = _fp8_ref(a, w, b, m, n, k)
    err = np.abs(dy.download().reshape(-1).astype(np.float64) - ref)
    tol = 2.0 ** -10 * asum + ulp
    assert np.all(err <= tol), float((err / tol).max())


# ---------------------------------------------------------------------------
# Every GEMM tile configuration (the context's GEMM_CFG override forces one per launch)
# ---------------------------------------------------------------------------

GEMM_CFGS = list(range(12))
CFG_SHAPES = [(1, 1, 128), (37, 100, 200), (300, 500, 384), (1100, 2304, 768), (513, 768, 3072)]


@pytest.fixture
def gemm_cfg(ctx):
    def force(cfg):
        ctx.set_tuning(D.TUNE_GEMM_CFG, cfg)
    yield force
    ctx.set_tuning(D.TUNE_GEMM_CFG, -1)


@pytest.mark.parametrize("cfg", GEMM_CFGS)
def test_gemm_every_config_int8(ctx, gemm_cfg, cfg):
    """INT32 accumulators (exact) and the per-token / per-channel epilogue
    (bit-exact) for every tile configuration, ragged and full shapes."""
    gemm_cfg(cfg)
    for m, n, k in CFG_SHAPES:
        say(f"cfg {cfg} int8 {m}x{n}x{k}")
        a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
        w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
        da, dw = D.DeviceBuffer.from_host(ctx, a), D.DeviceBuffer.from_host(ctx, w)
        dacc = D.DeviceBuffer.empty(ctx, (m, n), np.int32)
        D.matmul_int8_accum(ctx, da, dw, m, n, k, dacc)
        acc = a.astype(np.float64) @ w.astype(np.float64).T       # exact: |acc| < 2^53
        assert np.array_equal(dacc.download().astype(np.float64), acc), (cfg, m, n, k)
        sa = RNG.uniform(0.005, 0.05, m).astype(np.float32)
        sw = RNG.uniform(1e-4, 3e-4, n).astype(np.float32)
        b = RNG.normal(0, 0.01, n).astype(np.float32)
        dsa, dsw, db = (D.DeviceBuffer.from_host(ctx, v) for v in (sa, sw, b))
        dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        D.matmul_int8(ctx, da, dw, m, n, k, dsa, 1, 0.0, dsw, db, dy)
        want = ((acc * sa.astype(np.float64)[:, None]) * sw.astype(np.float64)[None, :]
                + b.astype(np.float64)[None, :]).astype(np.float32)
        assert _same_f32(dy.download(), want), (cfg, m, n, k)
        D.matmul_int8(ctx, da, dw, m, n, k, dsa, 0, 0.0, dsw, db, dy)   # per-tensor sa[0]
        want = ((acc * np.float64(sa[0])) * sw.astype(np.float64)[None, :]
                + b.astype(np.float64)[None, :]).astype(np.float32)
        assert _same_f32(dy.download(), want), (cfg, "per-tensor", m, n, k)


SKINNY_SHAPES = [(1, 1, 128), (1, 768, 3072), (32, 2304, 768), (17, 100, 200), (5, 300, 384),
                 (32, 768, 768), (4, 8320, 256), (9, 64, 4096)]


@pytest.mark.parametrize("dma", [0, 1])
def test_skinny_weight_paths(ctx, gemm_cfg, dma):
    """The skinny kernel (M <= 32) with its weight operand loaded per lane
    into registers (0) or copied into LDS as whole 128-byte lines (1): K
    split over workgroups (N = 768) and unsplit (one to sixteen waves), ragged
    N and K (K padded to the 128-byte step), a K range of 32 lines; INT32
    accumulators exact, the per-token and per-tensor epilogues and
    QLinearMatMul bit-exact."""
    gemm_cfg(10)
    ctx.set_tuning(D.TUNE_DECODE_DMA, dma)
    try:
        for m, n, k in SKINNY_SHAPES:
            say(f"skinny dma={dma} {m}x{n}x{k}")
            a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
            w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
            da, dw = D.DeviceBuffer.from_host(ctx, a), D.DeviceBuffer.from_host(ctx, w)
            dacc = D.DeviceBuffer.empty(ctx, (m, n), np.int32)
            D.matmul_int8_accum(ctx, da, dw, m, n, k, dacc)
            acc = a.astype(np.float64) @ w.astype(np.float64).T
            assert np.array_equal(dacc.download().astype(np.float64), acc), (dma, m, n, k)
            sa = RNG.uniform(0.005, 0.05, m).astype(np.float32)
            sw = RNG.uniform(1e-4, 3e-4, n).astype(np.float32)
            b = RNG.normal(0, 0.01, n).astype(np.float32)
            dsa, dsw, db = (D.DeviceBuffer.from_host(ctx, v) for v in (sa, sw, b))
            dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
            for stride in (1, 0):
                D.matmul_int8(ctx, da, dw, m, n, k, dsa, stride, 0.0, dsw, db, dy)
                s_a = sa.astype(np.float64)[:, None] if stride else np.float64(sa[0])
                want = ((acc * s_a) * sw.astype(np.float64)[None, :]
                        + b.astype(np.float64)[None, :]).astype(np.float32)
                assert _same_f32(dy.download(), want), (dma, stride, m, n, k)
            qsa, qsw = np.float32(0.02), np.float32(0.003)
            qsy = np.float32(np.sqrt(k) * 128 * 128 * qsa * qsw / 90.0)
            dq = D.DeviceBuffer.empty(ctx, (m, n), np.int8)
            _lib_check(D, "tkv_hip_dev_qlinear_matmul", ctx.handle, da.ptr, float(qsa), -3, dw.ptr,
                       float(qsw), 5, float(qsy), 7, dq.ptr, m, n, k, 0)
            bq = np.ascontiguousarray(w.reshape(n, k).T).reshape(-1).astype(np.int32)
            wantq = O.qlinear_matmul(a.reshape(-1).astype(np.int32), qsa, -3, bq, qsw, 5, qsy, 7,
                                     m * n, m, n, k)
            assert np.array_equal(dq.download().astype(np.int32).reshape(-1), wantq), (dma, m, n, k)
            for buf in (da, dw, dacc, dsa, dsw, db, dy, dq):
                buf.close()
    finally:
        ctx.set_tuning(D.TUNE_DECODE_DMA, -1)


@pytest.mark.parametrize("cfg", GEMM_CFGS)
def test_gemm_every_config_fp8(ctx, gemm_cfg, cfg):
    """Both FP8 policies under every tile configuration, to their stated
    bounds (reference products: 8 * 2^-24 * sum|p| + ulp; fast: 2^-10)."""
    gemm_cfg(cfg)
    for m, n, k in [(37, 100, 200), (300, 500, 384)]:
        say(f"cfg {cfg} fp8 {m}x{n}x{k}")
        a, w = _fp8_codes((m, k), False), _fp8_codes((n, k), False)
        b = RNG.normal(0, 1, n).astype(np.float32)
        da = D.DeviceBuffer.from_host(ctx, (a + 128).astype(np.uint8))
        dw = D.DeviceBuffer.from_host(ctx, (w + 128).astype(np.uint8))
        db = D.DeviceBuffer.from_host(ctx, b)
        dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        ref, asum, ulp = _fp8_ref(a, w, b, m, n, k)
        for fast, rel in ((False, 8 * 2.0 ** -24), (True, 2.0 ** -10)):
            D.matmul_fp8_e4m3(ctx, da, dw, m, n, k, None, 0, None, db, dy, fast=fast)
            err = np.abs(dy.download().reshape(-1).astype(np.float64) - ref)
            tol = rel * asum + ulp
            assert np.all(err <= tol), (cfg, fast, float((err / tol).max()))


# ---------------------------------------------------------------------------
# Resident weights + W8A8 linear (device pointers, no host sync in between)
# ---------------------------------------------------------------------------

def test_linear_forward_per_tensor(ctx):
    say("linear per-tensor (config 1)")
    x, w, b = _c1_inputs()
    m, n, k = 1024, 3072, 768
    dx, dw, db = (D.DeviceBuffer.from_host(ctx, v) for v in (x, w, b))
    lin = D.QuantizedLinear.from_float(ctx, dw, n, k, db, D.WEIGHT_INT8)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    lin.forward(dx, m, dy, D.ACT_PER_TENSOR)
    osw = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, n, k)], np.float32)
    owq = O.quantize_int8_per_channel(w, n, k, osw)
    opx = O.calibrate_minmax(x, 1)
    oxq = O.quantize_int8_symmetric(x, opx.scale)
    oy = O.matmul_int8_per_channel(oxq, owq, b, m, n, k, opx.scale, osw, threads=O.host_threads())
    assert _same_f32(dy.download(), oy)
    lin.close()


DECODE_SHAPES = [(m, n, k) for m in (1, 4, 16, 32)
                 for (n, k) in ((2304, 768), (3072, 768), (768, 3072))]


def test_linear_forward_per_token(ctx):
    """Config 5 decode shapes (skinny kernel, M <= 32; for N = 768 with K
    split over workgroups, whose partial-sum buffer each call must leave
    cleared for the next), the skinny kernel on N > 4096 columns and on K too
    short to split, then M = 33 (tiled) and the first shape again."""
    say("linear per-token (decode shapes)")
    for m, n, k in DECODE_SHAPES + [(4, 8320, 256), (4, 768, 256), (33, 768, 768),
                                    DECODE_SHAPES[0]]:
        x = _x(m * k, 11, 1.0)
        w = _x(n * k, 12, 0.02)
        b = _x(n, 13, 0.01)
        dx, dw, db = (D.DeviceBuffer.from_host(ctx, v) for v in (x, w, b))
        lin = D.QuantizedLinear.from_float(ctx, dw, n, k, db, D.WEIGHT_INT8)
        dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        lin.forward(dx, m, dy, D.ACT_PER_TOKEN)
        osw = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, n, k)], np.float32)
        owq = O.quantize_int8_per_channel(w, n, k, osw)
        oxq, osa = O.quantize_dynamic_int8_rowwise(x, m, k)
        acc = O.matmul_int8_accum(oxq, owq, m, n, k).reshape(m, n).astype(np.float64)
        want = (acc * osa.astype(np.float64)[:, None] * osw.astype(np.float64)[None, :]
                + b.astype(np.float64)[None, :]).astype(np.float32)
        assert _same_f32(dy.download(), want), (m, n, k)
        lin.close()


def _per_token_want(x, w, b, m, n, k):
    osw = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, n, k)], np.float32)
    owq = O.quantize_int8_per_channel(w, n, k, osw)
    oxq, osa = O.quantize_dynamic_int8_rowwise(x, m, k)
    acc = O.matmul_int8_accum(oxq, owq, m, n, k).reshape(m, n).astype(np.float64)
    return (acc * osa.astype(np.float64)[:, None] * osw.astype(np.float64)[None, :]
            + b.astype(np.float64)[None, :]).astype(np.float32)


DECODE_EDGE = [(1, 100, 64), (3, 17, 128), (5, 33, 192), (17, 200, 1024), (31, 2304, 768),
               (32, 768, 3072), (2, 768, 3072), (8, 3072, 768), (20, 100, 64), (24, 130, 128),
               (9, 300, 448)]


@pytest.mark.parametrize("rg,dma", [(None, None), (1, None), (3, None), (16, None),
                                    (None, 0), (None, 1), (3, 1)])
def test_decode_linear_edge_cases(ctx, rg, dma):
    """The one-kernel decode linear (per-token quantize + INT8 GEMM +
    epilogue, M <= 32): ragged row groups and column blocks, one to sixteen
    waves, workgroups of several column blocks above 16 tokens (with fewer
    waves than blocks at K = 64 and 128), a zero row (scale floor), a row
    holding NaN (skipped by the absmax, coded 0), an outlier row; forced
    row-group sizes; both weight paths forced on every shape (registers, and
    whole lines through LDS, whose DMA count per wave is 4 at K = 192 and
    shares lines between waves); and a misaligned x, which takes the
    two-kernel path.  Bit-exact."""
    ctx.set_tuning(D.TUNE_DECODE_GROUP, -1 if rg is None else rg)
    ctx.set_tuning(D.TUNE_DECODE_DMA, -1 if dma is None else dma)
    try:
        _decode_edge_cases(ctx, rg)
    finally:
        ctx.set_tuning(D.TUNE_DECODE_GROUP, -1)
        ctx.set_tuning(D.TUNE_DECODE_DMA, -1)


def _decode_edge_cases(ctx, rg):
    for m, n, k in DECODE_EDGE:
        say(f"decode linear rg={rg} {m}x{n}x{k}")
        x = _x(m * k, 31 + m, 1.0).reshape(m, k)
        x[0] = 0.0
        if m > 1:
            x[1, 5] = np.nan
        if m > 2:
            x[2, k // 3] = 3.0e4
        x = x.reshape(-1)
        w = _x(n * k, 32, 0.02)
        w[:k] = 0.0                                     # an all-zero weight row
        b = _x(n, 33, 0.01)
        dw, db = D.DeviceBuffer.from_host(ctx, w), D.DeviceBuffer.from_host(ctx, b)
        lin = D.QuantizedLinear.from_float(ctx, dw, n, k, db, D.WEIGHT_INT8)
        dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
        want = _per_token_want(x, w, b, m, n, k)
        dx = D.DeviceBuffer.from_host(ctx, x)
        lin.forward(dx, m, dy, D.ACT_PER_TOKEN)
        assert _same_f32(dy.download(), want), (rg, m, n, k)
        if rg is None and k % 128 == 0:
            # x one float past a 16-byte boundary: the two-kernel fallback
            dxo = D.DeviceBuffer.from_host(ctx, np.concatenate([np.zeros(1, np.float32), x]))
            lin.forward(dxo.ptr + 4, m, dy, D.ACT_PER_TOKEN)
            assert _same_f32(dy.download(), want), ("misaligned", m, n, k)
            dxo.close()
        for buf in (dx, dw, db, dy):
            buf.close()
        lin.close()


@pytest.mark.parametrize("cfg", GEMM_CFGS)
def test_qlinear_matmul_device_every_config(ctx, gemm_cfg, cfg):
    """Device QLinearMatMul (fused requantizing epilogue, int8 out) on every
    GEMM configuration, including the skinny kernel (M <= 32; at N = 768
    with K split over workgroups), bit-exact."""
    gemm_cfg(cfg)
    # zero points: both set; zpa = 0 (no W sums needed); zpw = 0 (no A sums);
    # both 0 (no pre-pass at all); zpw = 0 with |zpa| large enough for the f64
    # correction path at K = 768.  M > 32 with one tile or few K slices per
    # workgroup forms the row sums inside the GEMM (split over the waves on
    # the warp-specialised configurations); launches with several tiles per
    # workgroup and many slices (the pre-pass) are in
    # test_qlinear_sums_tile_runs.
    cases = [((37, 100, 200), (-3, 5, 7)), ((1024, 768, 768), (-3, 5, 7)),
             ((16, 2304, 768), (-3, 5, 7)), ((16, 768, 3072), (-3, 5, 7)),
             ((37, 100, 200), (0, 5, 7)), ((37, 100, 200), (-3, 0, 7)),
             ((1024, 768, 768), (0, 0, -2)), ((64, 96, 768), (30000, 0, 3)),
             ((64, 96, 768), (0, -30000, 3)), ((1024, 768, 3072), (-3, 5, 7)),
             ((1024, 768, 3072), (0, 5, 7))]
    for (m, n, k), (zpa, zpw, zpy) in cases:
        say(f"dev qlinear cfg={cfg} {m}x{n}x{k} zp={zpa},{zpw},{zpy}")
        a = RNG.integers(-128, 128, m * k).astype(np.int8)
        w = RNG.integers(-128, 128, n * k).astype(np.int8)   # [N, K] = B transposed
        sa, sw = np.float32(0.02), np.float32(0.003)
        sy = np.float32(np.sqrt(k) * 128 * 128 * sa * sw / 90.0)
        da, dw = D.DeviceBuffer.from_host(ctx, a), D.DeviceBuffer.from_host(ctx, w)
        dy = D.DeviceBuffer.empty(ctx, (m, n), np.int8)
        _lib_check(D, "tkv_hip_dev_qlinear_matmul", ctx.handle, da.ptr, float(sa), zpa, dw.ptr,
                   float(sw), zpw, float(sy), zpy, dy.ptr, m, n, k, 0)
        b = np.ascontiguousarray(w.reshape(n, k).T).reshape(-1).astype(np.int32)
        want = O.qlinear_matmul(a.astype(np.int32), sa, zpa, b, sw, zpw, sy, zpy, m * n, m, n, k)
        got = dy.download().astype(np.int32).reshape(-1)
        assert np.array_equal(got, want), (cfg, m, n, k, int(np.sum(got != want)))


def test_qlinear_sums_tile_runs(ctx, gemm_cfg):
    """QLinearMatMul on launches where workgroups run several tiles.  Row /
    column sums split over the waves of the warp-specialised kernel and
    exchanged through LDS at each tile's end (the two LDS areas alternate by
    tile): 264 tiles of cfg 2 on 256 CUs, more on cfg 5 / 8, with one K slice
    (the exchange's first and last slice coincide) and three; both zero-point
    sums, and W sums only.  K = 896 gives 14 slices per workgroup: the sums
    come from the pre-pass.  Bit-exact against the oracle."""
    for (m, n, k), (zpa, zpw, zpy) in [((4224, 1536, 128), (-3, 5, 7)),
                                       ((4224, 1536, 384), (-3, 5, 7)),
                                       ((4224, 1536, 384), (6, 0, -2)),
                                       ((4224, 1536, 896), (-3, 5, 7))]:
        a = RNG.integers(-128, 128, m * k).astype(np.int8)
        w = RNG.integers(-128, 128, n * k).astype(np.int8)
        sa, sw = np.float32(0.02), np.float32(0.003)
        sy = np.float32(np.sqrt(k) * 128 * 128 * sa * sw / 90.0)
        b = np.ascontiguousarray(w.reshape(n, k).T).reshape(-1).astype(np.int32)
        want = O.qlinear_matmul(a.astype(np.int32), sa, zpa, b, sw, zpw, sy, zpy, m * n, m, n, k)
        da, dw = D.DeviceBuffer.from_host(ctx, a), D.DeviceBuffer.from_host(ctx, w)
        dy = D.DeviceBuffer.empty(ctx, (m, n), np.int8)
        for cfg in (-1, 2, 5, 8):
            say(f"qlinear tile runs cfg={cfg} {m}x{n}x{k} zp={zpa},{zpw},{zpy}")
            gemm_cfg(cfg)
            _lib_check(D, "tkv_hip_dev_qlinear_matmul", ctx.handle, da.ptr, float(sa), zpa,
                       dw.ptr, float(sw), zpw, float(sy), zpy, dy.ptr, m, n, k, 0)
            got = dy.download().astype(np.int32).reshape(-1)
            assert np.array_equal(got, want), (cfg, m, n, k, int(np.sum(got != want)))
        for buf in (da, dw, dy):
            buf.close()


def _lib_check(D, name, *args):
    from tokenvector.inference_amd import _lib
    _lib.check(getattr(_lib.lib(), name)(*args))


# ---------------------------------------------------------------------------
# stream capture (tkv_hip_capture_begin / capture_end / graph_launch)
# ---------------------------------------------------------------------------

def test_graph_capture_replays(hip):
    """A captured layer (dynamic quantize, an INT8 GEMM whose K needs the
    zero-padded operand repack, a byte fill) replays to the eager results bit
    for bit: three replays, each after new input values, other eager work and
    a synchronization.  A call that would grow a workspace inside a capture is
    refused on the host, and the stream runs eagerly again afterwards."""
    say("graph capture replays")
    ctx = D.Context(0)  # fresh workspaces: the refusal below depends on their sizes
    m, n, k = 300, 200, 200
    w = _x(n * k, 63, 0.05)
    sw = np.array([q.scale for q in O.calibrate_per_channel_minmax(w, n, k)], np.float32)
    wq = O.quantize_int8_per_channel(w, n, k, sw).astype(np.int8)
    dw, dsw = D.DeviceBuffer.from_host(ctx, wq), D.DeviceBuffer.from_host(ctx, sw)
    db = D.DeviceBuffer.from_host(ctx, _x(n, 64, 0.01))
    dx = D.DeviceBuffer.empty(ctx, (m, k), np.float32)
    qa = D.DeviceBuffer.empty(ctx, (m, k), np.int8)
    dy = D.DeviceBuffer.empty(ctx, (m, n), np.float32)
    fill = D.DeviceBuffer.empty(ctx, 1000, np.uint8)
    p = D.params_buffer(ctx)
    other_x = D.DeviceBuffer.from_host(ctx, _x(4099, 65, 1.0))
    other_q = D.DeviceBuffer.empty(ctx, 4099, np.int8)
    other_p = D.params_buffer(ctx)

    def layer():
        D.quantize_int8_dynamic_tensor(ctx, dx, m * k, qa, p)
        D.matmul_int8(ctx, qa, dw, m, n, k, p.ptr, 0, 0.0, dsw, db, dy)
        D.memset(ctx, fill.ptr + 3, 0x5A, 990)

    inputs = [_x(m * k, 70 + i, 1.0 + i) for i in range(3)]
    want = []
    for x in inputs:
        dx.upload(x)
        D.memset(ctx, fill, 0, 1000)
        layer()
        ctx.synchronize()
        want.append((qa.download(), dy.download(), fill.download()))
    f = np.zeros(1000, np.uint8)
    f[3:993] = 0x5A
    assert np.array_equal(want[0][2], f)

    with D.Graph(ctx) as g:
        layer()
    for rep in range(2):
        for x, (wqa, wy, wf) in zip(inputs, want):
            dx.upload(x)
            D.quantize_int8_dynamic_tensor(ctx, other_x, 4099, other_q, other_p)
            D.memset(ctx, fill, 0, 1000)
            D.memset(ctx, qa, 0, m * k)
            ctx.synchronize()
            g.launch()
            ctx.synchronize()
            assert np.array_equal(qa.download(), wqa), rep
            assert np.array_equal(dy.download(), wy), rep
            assert np.array_equal(fill.download(), wf), rep
    g.close()

    # K = 300 pads to 384: 4100 x 384 bytes outgrows the 1 MiB repack slot
    big_a = D.DeviceBuffer.empty(ctx, (4100, 300), np.int8)
    big_w = D.DeviceBuffer.empty(ctx, (n, 300), np.int8)
    big_y = D.DeviceBuffer.empty(ctx, (4100, n), np.float32)
    with pytest.raises((ValueError, RuntimeError), match="stream capture"):
        with D.Graph(ctx) as bad:
            D.matmul_int8(ctx, big_a, big_w, 4100, n, 300, p.ptr, 0, 0.0, dsw, db, big_y)
    bad.close()
    dx.upload(inputs[1])
    layer()
    ctx.synchronize()
    assert np.array_equal(dy.download(), want[1][1])
    ctx.close()


def test_graph_replays_calibrators(hip):
    """calibrate_minmax (finalized by its last partials workgroup), KL,
    percentile (symmetric, with the staged third radix pass, and asymmetric)
    and MSE captured in one graph.  Each finishes in its last workgroup, on
    arrival counters and a histogram that every call leaves zero, so replays
    after new input values, eager calibrator calls on other data and
    synchronizations give the eager results, which equal the oracle's."""
    say("graph replays calibrators")
    ctx = D.Context(0)
    n = 8192 * 96
    dx = D.DeviceBuffer.empty(ctx, n, np.float32)
    ps = [D.params_buffer(ctx) for _ in range(5)]

    def calib():
        D.calibrate_minmax(ctx, dx, n, 1, ps[0])
        D.calibrate_kl(ctx, dx, n, ps[1])
        D.calibrate_percentile(ctx, dx, n, ps[2], 99.9, 1)
        D.calibrate_percentile(ctx, dx, n, ps[3], 50.0, 0)
        D.calibrate_mse(ctx, dx, n, ps[4], 20)

    inputs = [O.add_outliers(_x(n, 80 + i, 1.0 + i), 0.001, 3, 4, 20.0) for i in range(3)]
    want = []
    for x in inputs:
        dx.upload(x)
        calib()
        ctx.synchronize()
        want.append([p.download().tobytes() for p in ps])
    x = inputs[0]
    dx.upload(x)
    calib()
    assert _same_qp(D.read_params(ps[0]), O.calibrate_minmax(x, 1))
    assert _same_qp(D.read_params(ps[1]), O.calibrate_kl(x))
    assert _same_qp(D.read_params(ps[2]), O.calibrate_percentile(x, 99.9, 1))
    assert _same_qp(D.read_params(ps[3]), O.calibrate_percentile(x, 50.0, 0))
    assert _same_qp(D.read_params(ps[4]), O.calibrate_mse(x, 20))

    other = D.DeviceBuffer.from_host(ctx, _x(5000, 90, 1.0))
    op = D.params_buffer(ctx)
    with D.Graph(ctx) as g:
        calib()
    for rep in range(2):
        for x, w in zip(inputs, want):
            dx.upload(x)
            D.calibrate_kl(ctx, other, 5000, op)
            D.calibrate_percentile(ctx, other, 5000, op, 99.0, 1)
            D.calibrate_minmax(ctx, other, 5000, 0, op)
            ctx.synchronize()
            for p in ps:
                D.memset(ctx, p, 0, p.nbytes)
            g.launch()
            ctx.synchronize()
            assert [p.download().tobytes() for p in ps] == w, rep
    g.close()


def test_graph_replays_single_pass_quantize(hip):
    """The single-pass calibrate + quantize (a 100 MB activation: one
    workgroup per CU and a grid barrier whose slots advance by one generation
    per launch) inside a captured graph: three replays over new inputs, with
    eager single-pass calls of another size between them, each equal to the
    eager result bit for bit."""
    say("graph replays of the single-pass quantize")
    ctx = D.Context(0)
    n = 8192 * 3072
    dx = D.DeviceBuffer.empty(ctx, n, np.float32)
    dq = D.DeviceBuffer.empty(ctx, n, np.int8)
    p = D.params_buffer(ctx)
    other = _res_input(2 ** 24 + 12, 91)
    dox = D.DeviceBuffer.from_host(ctx, other)
    doq = D.DeviceBuffer.empty(ctx, other.size, np.int8)
    dop = D.params_buffer(ctx)
    inputs = [_res_input(n, 80 + i) for i in range(3)]
    want = []
    for x in inputs:
        dx.upload(x)
        D.quantize_int8_dynamic_tensor(ctx, dx, n, dq, p)
        ctx.synchronize()
        want.append((D.read_params(p).scale, dq.download()))
    wp = O.calibrate_minmax(inputs[0], 1)
    assert _same_f32([want[0][0]], [wp.scale])
    assert np.array_equal(want[0][1].astype(np.int32), O.quantize_int8_symmetric(inputs[0], wp.scale))
    with D.Graph(ctx) as g:
        D.quantize_int8_dynamic_tensor(ctx, dx, n, dq, p)
    for x, (ws, wq) in zip(inputs, want):
        dx.upload(x)
        D.quantize_int8_dynamic_tensor(ctx, dox, other.size, doq, dop)
        D.memset(ctx, dq, 0, n)
        ctx.synchronize()
        g.launch()
        ctx.synchronize()
        assert _same_f32([D.read_params(p).scale], [ws])
        assert np.array_equal(dq.download(), wq)
    g.close()
    op = O.calibrate_minmax(other, 1)
    assert _same_f32([D.read_params(dop).scale], [op.scale])
    assert np.array_equal(doq.download().astype(np.int32), O.quantize_int8_symmetric(other, op.scale))
    ctx.close()


def test_graph_survives_workspace_growth(hip):
    """A graph captured over a call that repacks its operands into workspace
    still replays correctly after a larger eager call has grown those
    workspaces: the old buffers stay alive (retired) while the graph does,
    and are freed with it."""
    say("graph replay after workspace growth")
    ctx = D.Context(0)
    m, n, k = 64, 96, 200                       # K = 200 repacks into slots 2 / 3
    a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    da, dw = D.DeviceBuffer.from_host(ctx, a), D.DeviceBuffer.from_host(ctx, w)
    dacc = D.DeviceBuffer.empty(ctx, (m, n), np.int32)
    D.matmul_int8_accum(ctx, da, dw, m, n, k, dacc)
    ctx.synchronize()
    want = (a.astype(np.int64) @ w.astype(np.int64).T)
    assert np.array_equal(dacc.download(), want)
    with D.Graph(ctx) as g:
        D.matmul_int8_accum(ctx, da, dw, m, n, k, dacc)
    assert ctx.retired_buffers() == 0
    # K = 300 pads to 384: 4100 x 384 bytes outgrows the 1 MiB repack slot
    bm, bk = 4100, 300
    ba = RNG.integers(-127, 128, (bm, bk)).astype(np.int8)
    bw = RNG.integers(-127, 128, (n, bk)).astype(np.int8)
    dba, dbw = D.DeviceBuffer.from_host(ctx, ba), D.DeviceBuffer.from_host(ctx, bw)
    dbacc = D.DeviceBuffer.empty(ctx, (bm, n), np.int32)
    D.matmul_int8_accum(ctx, dba, dbw, bm, n, bk, dbacc)
    ctx.synchronize()
    assert ctx.retired_buffers() >= 1
    assert np.array_equal(dbacc.download(), ba.astype(np.int64) @ bw.astype(np.int64).T)
    for rep in range(3):
        D.memset(ctx, dacc, 0, m * n * 4)
        da.upload(np.roll(a, rep, axis=0))
        ctx.synchronize()
        g.launch()
        ctx.synchronize()
        assert np.array_equal(dacc.download(), np.roll(want, rep, axis=0)), rep
    g.close()
    assert ctx.retired_buffers() == 0
    D.matmul_int8_accum(ctx, da, dw, m, n, k, dacc)
    ctx.synchronize()
    assert np.array_equal(dacc.download(), np.roll(want, 2, axis=0))
    ctx.close()
