"""Pins the CPU oracle (oracle/tkv_oracle.c) before it is trusted as the
parity checker.  Each check is independent of the oracle's own code:

* the reference's own asserts (tv/tests/gap_tests.tkv:158-240,
  tv/tests/inference_tests.tkv:896-948) live in test_golden.py, driven by
  tests/golden/reference_kats.json;
* library routines (numpy IEEE float32 arithmetic, numpy int64 matmul,
  numpy rint, torch float8 casts, Python Fractions);
* exhaustive comparison with an independently formulated encoder.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------------------
# f32_bits.tkv
# ---------------------------------------------------------------------------

def _sample_f32_bits(n):
    bits = RNG.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    special = np.array([0x00000001, 0x007FFFFF, 0x00800000, 0x3F800000, 0x7F7FFFFF,
                        0x80000001, 0x807FFFFF, 0xFF7FFFFF, 0x3EFFFFFF, 0x4B7FFFFF], np.uint32)
    bits = np.concatenate([bits, special])
    exp = (bits >> 23) & 0xFF
    return bits[exp != 255]


def test_f64_to_f32_bits_is_ieee_bit_pattern():
    for b in _sample_f32_bits(3000):
        x = float(np.array([b], np.uint32).view(np.float32)[0])
        want = int(b)
        if x == 0.0:                      # x == 0.0 returns 0 (f32_bits.tkv:19-20)
            want = 0
        elif (int(b) & 0x7FFFFFFF) == 1:  # 2^-149: sh = e + 149 = 0 hits `sh <= 0` (:38-39)
            want = int(b) & 0x80000000
        assert O.f64_to_f32_bits(x) == want, hex(int(b))


def test_f32_bits_to_f64_is_ieee_value():
    for b in _sample_f32_bits(3000):
        x = float(np.array([b], np.uint32).view(np.float32)[0])
        got = O.f32_bits_to_f64(int(b))
        assert got == x or (x == 0.0 and got == 0.0), hex(int(b))
    # exponent 255 yields +-2^129 whatever the mantissa (f32_bits.tkv:68-69)
    assert O.f32_bits_to_f64(0x7F800001) == 2.0 ** 129
    assert O.f32_bits_to_f64(0xFFC00000) == -(2.0 ** 129)


def test_rne_rshift_bruteforce():
    for s in range(0, 15):
        for v in range(0, 4096, 3):
            q = Fraction(v, 2 ** s)
            fl = q.numerator // q.denominator
            rem = q - fl
            want = fl + (1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1) else 0)
            assert O.rne_rshift(v, s) == want, (v, s)


# ---------------------------------------------------------------------------
# e4m3 codec
# ---------------------------------------------------------------------------

def _ocp_e4m3_value(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 15, code & 7
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1 + m / 8) * 2.0 ** (e - 7)


def test_e4m3_decode_all_codes():
    """OCP e4m3fn values except the reference decoder's fixed departures:
    subnormals decode to half (types.tkv:216-222 normalises with exponent
    127 - bias - n), 0x7F/0xFF are +-inf (f32_bits_to_f64 ignores the
    mantissa at exponent 255) and 0x80 is +0.0 (0.0 - 0.0)."""
    for c in range(256):
        got = O.fp8_e4m3_decode(c)
        e, m = (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            assert np.isinf(got) and (got < 0) == bool(c & 0x80)
        elif e == 0 and m == 0:
            assert got == 0.0 and not np.signbit(got)
        elif e == 0:
            assert got == np.float32(_ocp_e4m3_value(c) / 2), hex(c)
        else:
            assert got == np.float32(_ocp_e4m3_value(c)), hex(c)


def test_e4m3_normal_decode_matches_torch():
    torch = pytest.importorskip("torch")
    codes = [c for c in range(256) if ((c >> 3) & 15) not in (0,) and (c & 0x7F) != 0x7F]
    t = torch.tensor(codes, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    for c, v in zip(codes, t):
        assert O.fp8_e4m3_decode(c) == v, hex(c)


def test_e4m3_spec_encoder_matches_torch():
    """The independent spec encoder agrees with torch's e4m3fn RNE cast
    wherever the reference does not deviate (|x| < 240, outside the
    subnormal clamp band [7.5 * 2^-9, 2^-6), x != -0.0)."""
    torch = pytest.importorskip("torch")
    x = np.concatenate([
        RNG.normal(0, 1, 20000), RNG.normal(0, 60, 20000), RNG.normal(0, 0.01, 20000),
        np.arange(-239.5, 239.5, 0.0625),
    ]).astype(np.float32)
    band = (np.abs(x) >= 7.5 * 2.0 ** -9) & (np.abs(x) < 2.0 ** -6)
    keep = (np.abs(x) < 240) & ~band & ~((x == 0) & np.signbit(x))
    x = x[keep]
    tb = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    for v, b in zip(x[::7], tb[::7]):
        assert O.spec_e4m3_encode(float(v)) == int(b), float(v)


def test_e4m3_encode_exhaustive_vs_spec():
    """Every finite f32 bit pattern (exponent fields 0..254, both signs):
    the restated reference encoder equals the independent spec encoder."""
    bad, first = O.e4m3_exhaustive(0, 254)
    assert bad == 0, hex(first)


def test_e4m3_encode_deviations():
    # Appendix of the reference's encoder behaviour (types.tkv:176-183, f32_bits.tkv:19-20)
    assert O.fp8_e4m3_encode(247.99) == 0x77
    assert O.fp8_e4m3_encode(248.0) == 0x7E and O.fp8_e4m3_encode(-300.0) == 0xFE
    assert O.fp8_e4m3_encode(0.0136) == 0x07          # OCP would give 0x08
    assert O.fp8_e4m3_encode(-0.0) == 0x00
    assert O.fp8_e4m3_encode(float("nan")) == 0x38    # NaN -> bits of 1.0


# ---------------------------------------------------------------------------
# engine.tkv calibrate / quantize / dequantize
# ---------------------------------------------------------------------------

def test_calibrate_symmetric_closed_form():
    for scale in (1e-3, 1.0, 37.0):
        x = (RNG.normal(0, scale, 5000)).astype(np.float32)
        p = O.calibrate_minmax(x, 1)
        am = np.float32(np.max(np.abs(x)))
        assert p.scale == am / np.float32(127.0)      # numpy IEEE f32 division
        assert p.min_val == -am and p.max_val == am and p.zero_point == 0
    p = O.calibrate_minmax(np.zeros(8, np.float32), 1)
    assert p.scale == np.float32(1e-8 / 127.0)
    p = O.quant_identity()
    assert p.scale == 1.0 and p.max_val == np.float32(3.4028234663852886e38)


def test_calibrate_asymmetric():
    p = O.calibrate_minmax(np.array([0.0, 1.0, 2.0], np.float32), 0)
    assert p.scale == np.float32(2.0 / 255.0) and p.zero_point == -128
    x = RNG.normal(0.5, 2.0, 1000).astype(np.float32)
    p = O.calibrate_minmax(x, 0)
    mn, mx = float(x.min()), float(x.max())
    sc = (mx - mn) / 255.0
    zp = int(np.clip(np.rint(-mn / sc) - 128, -128, 127))
    assert p.scale == np.float32(sc) and p.zero_point == zp
    assert p.min_val == np.float32(mn) and p.max_val == np.float32(mx)
    # a zero extreme keeps the first zero's sign (first occurrence wins)
    assert np.signbit(O.calibrate_minmax(np.array([3.0, -0.0, 0.0], np.float32), 0).min_val)
    assert not np.signbit(O.calibrate_minmax(np.array([3.0, 0.0, -0.0], np.float32), 0).min_val)


def test_calibrate_per_channel_equals_rowwise():
    w = RNG.normal(0, 0.02, (7, 33)).astype(np.float32)
    ps = O.calibrate_per_channel_minmax(w, 7, 33, 1)
    for r in range(7):
        assert ps[r] == O.calibrate_minmax(w[r], 1)
        assert ps[r].scale == np.float32(np.max(np.abs(w[r]))) / np.float32(127)
    with pytest.raises(ValueError):
        O.calibrate_per_channel_minmax(w, 0, 33)
    with pytest.raises(ValueError):
        O.calibrate_per_channel_minmax(w, 8, 33)


def _rne_clamp(v, lo=-127, hi=127):
    return np.clip(np.rint(v), lo, hi).astype(np.int64)


def test_quantize_symmetric_properties():
    x = RNG.normal(0, 1, 20000).astype(np.float32)
    p = O.calibrate_minmax(x, 1)
    q = O.quantize_int8_symmetric(x, p.scale)
    inv = np.float64(np.float32(1.0) / p.scale)         # f32 reciprocal (primary)
    assert np.array_equal(q, _rne_clamp(x.astype(np.float64) * inv))
    assert np.abs(q).max() <= 127
    qa = O.quantize_int8_symmetric(x, p.scale, O.ALTERNATE)
    assert np.array_equal(qa, _rne_clamp(x.astype(np.float64) * (1.0 / np.float64(p.scale))))
    # ties to even: scale 2^-4 makes x * inv = k + 0.5 exactly
    k = np.arange(-20, 20)
    xt = ((k + 0.5) / 16.0).astype(np.float32)
    qt = O.quantize_int8_symmetric(xt, 2.0 ** -4)
    assert np.all(qt % 2 == 0) and np.all(np.abs(qt - (k + 0.5)) == 0.5)
    # clamp, non-finite inputs, scale floor
    q = O.quantize_int8_symmetric([1e30, -1e30, np.inf, -np.inf, np.nan], 0.5)
    assert list(q) == [127, -127, 127, -127, 0]
    q = O.quantize_int8_symmetric([1e-7, -3e-7, 2e-6], 1e-9)   # inv = 1e8
    assert list(q) == [10, -30, 127]


def test_quantize_per_channel_and_dynamic():
    w = RNG.normal(0, 0.02, (16, 96)).astype(np.float32)
    sc = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, 16, 96)], np.float32)
    q = O.quantize_int8_per_channel(w, 16, 96, sc).reshape(16, 96)
    inv = 1.0 / np.maximum(sc.astype(np.float64), 1e-8)
    assert np.array_equal(q, _rne_clamp(w.astype(np.float64) * inv[:, None]))
    x = RNG.normal(0, 1, (9, 40)).astype(np.float32)
    x[3] = 0.0
    qd, so = O.quantize_dynamic_int8_rowwise(x, 9, 40)
    am = np.maximum(np.abs(x).max(axis=1).astype(np.float64), 1e-8)
    sc64 = am / 127.0
    assert np.array_equal(so, sc64.astype(np.float32))
    assert np.array_equal(qd.reshape(9, 40), _rne_clamp(x.astype(np.float64) * (1.0 / sc64)[:, None]))


def test_dequantize_closed_form():
    q = RNG.integers(-127, 128, 1000).astype(np.int32)
    s = np.float32(0.0137)
    assert np.array_equal(O.dequantize_int8_symmetric(q, s), q.astype(np.float32) * s)
    sc = RNG.uniform(1e-4, 1e-2, 10).astype(np.float32)
    qq = RNG.integers(-127, 128, (10, 100)).astype(np.int32)
    assert np.array_equal(O.dequantize_int8_per_channel(qq, 10, 100, sc).reshape(10, 100),
                          qq.astype(np.float32) * sc[:, None])


# ---------------------------------------------------------------------------
# matmul.tkv
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 5, 31), (7, 4, 33), (16, 16, 64), (5, 9, 200)])
def test_int8_accumulators_bruteforce(m, n, k):
    a = RNG.integers(-128, 128, (m, k)).astype(np.int32)
    w = RNG.integers(-128, 128, (n, k)).astype(np.int32)
    acc = O.matmul_int8_accum(a, w, m, n, k).reshape(m, n)
    assert np.array_equal(acc, a.astype(np.int64) @ w.astype(np.int64).T)


def _ulp32(v):
    v = np.abs(np.float32(v))
    return float(np.spacing(v)) if v > 0 else 2.0 ** -149


def test_int8_per_channel_epilogue_exact():
    m, n, k = 6, 11, 64
    a = RNG.integers(-127, 128, (m, k)).astype(np.int32)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int32)
    sa = np.float32(0.0213)
    sw = RNG.uniform(1e-4, 3e-4, n).astype(np.float32)
    b = RNG.normal(0, 0.01, n).astype(np.float32)
    y = O.matmul_int8_per_channel(a, w, b, m, n, k, sa, sw).reshape(m, n)
    acc = a.astype(np.int64) @ w.astype(np.int64).T
    for i in range(m):
        for j in range(n):
            exact = Fraction(int(acc[i, j])) * Fraction(float(sa)) * Fraction(float(sw[j])) + Fraction(float(b[j]))
            mag = abs(Fraction(int(acc[i, j])) * Fraction(float(sa)) * Fraction(float(sw[j]))) + abs(Fraction(float(b[j])))
            err = abs(Fraction(float(y[i, j])) - exact)
            assert err <= Fraction(_ulp32(y[i, j])) / 2 + mag * Fraction(3, 2 ** 53)
    # permuting the channel scales / bias permutes output columns
    perm = RNG.permutation(n)
    y2 = O.matmul_int8_per_channel(a, w[perm], b[perm], m, n, k, sa, sw[perm]).reshape(m, n)
    assert np.array_equal(y2, y[:, perm])
    # no bias (len(pbias) == 0)
    y0 = O.matmul_int8_per_channel(a, w, None, m, n, k, sa, sw).reshape(m, n)
    assert np.array_equal(y0, (acc.astype(np.float64) * float(sa) * sw.astype(np.float64)).astype(np.float32))
    with pytest.raises(ValueError):
        O.matmul_int8_per_channel(a, w, b, m, n, k, sa, sw[:-1])


def test_int8_symmetric_epilogue():
    m, n, k = 5, 7, 96
    a = RNG.integers(-127, 128, (m, k)).astype(np.int32)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int32)
    sa, swt = np.float32(0.011), np.float32(0.00031)
    b = RNG.normal(0, 0.01, n).astype(np.float32)
    y = O.matmul_int8_symmetric(a, w, b, m, n, k, sa, swt).reshape(m, n)
    s = sa * swt                                       # numpy f32 multiply
    acc = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(y, (acc.astype(np.float64) * np.float64(s) + b.astype(np.float64)).astype(np.float32))


def _dec_table():
    t = np.zeros(256, np.float64)
    for c in range(256):
        e, m = (c >> 3) & 15, c & 7
        t[c] = _ocp_e4m3_value(c) / (2.0 if e == 0 else 1.0)
    return t


def test_fp8_gemm_exact_sum():
    m, n, k = 4, 6, 160
    codes = [c for c in range(256) if (c & 0x7F) != 0x7F]
    a = (RNG.choice(codes, (m, k)) - 128).astype(np.int32)
    w = (RNG.choice(codes, (n, k)) - 128).astype(np.int32)
    b = RNG.normal(0, 1, n).astype(np.float32)
    y = O.matmul_fp8_e4m3(a, w, b, m, n, k).reshape(m, n)
    t = _dec_table()
    da, dw = t[a + 128], t[w + 128]
    for i in range(m):
        for j in range(n):
            s = sum(Fraction(float(p)) for p in da[i] * dw[j])  # products exact in f64
            want = np.float32(float(s + Fraction(float(b[j]))))
            assert y[i, j] == want
    acc, asum = O.matmul_fp8_e4m3_exact(a, w, m, n, k)
    assert np.array_equal(acc.astype(np.float64) * 2.0 ** -20, (da @ dw.T).reshape(-1))
    assert np.allclose(asum, (np.abs(da) @ np.abs(dw).T).reshape(-1), rtol=1e-12)


def test_fp8_quantize_codes():
    x = RNG.normal(0, 50, 3000).astype(np.float32)
    q = O.quantize_fp8_e4m3(x)
    assert np.array_equal(q + 128, [O.spec_e4m3_encode(float(v)) for v in x])
    d = O.dequantize_fp8_e4m3(q)
    assert np.array_equal(d, _dec_table()[q + 128].astype(np.float32))


# ---------------------------------------------------------------------------
# session.tkv nodes
# ---------------------------------------------------------------------------

def test_matmul_integer_bounds_semantics():
    m, n, k = 5, 7, 9
    a = RNG.integers(-128, 128, m * k - 4).astype(np.int32)   # short A: tail reads 0
    b = RNG.integers(-128, 128, k * n).astype(np.int32)
    y = O.matmul_integer(a, b, m * n - 3, m, n, k)            # short Y: tail dropped
    ap = np.zeros(m * k, np.int64)
    ap[: a.size] = a
    want = (ap.reshape(m, k) @ b.astype(np.int64).reshape(k, n)).reshape(-1)
    assert np.array_equal(y, want[: m * n - 3])


def _qlinear_numpy(a, sa, zpa, b, sw, zpw, sy, zpy, ny, m, n, k, recipe):
    """Independent restatement with numpy: in-range reads as (code - zp),
    out-of-range as 0, int64 matmul, f64 multiply, numpy rint (half even)."""
    a, b = np.asarray(a, np.int64), np.asarray(b, np.int64)
    av = np.zeros((m, k), np.int64)
    bv = np.zeros((k, n), np.int64)
    ia = np.arange(m * k).reshape(m, k)
    ib = np.arange(k * n).reshape(k, n)
    av[ia < a.size] = a[ia[ia < a.size]] - zpa
    bv[ib < b.size] = b[ib[ib < b.size]] - zpw
    acc = av @ bv
    if recipe == O.PRIMARY:
        mult = np.float64(np.float32(sa)) * np.float64(np.float32(sw)) / (
            np.float64(np.float32(sy)) if np.float32(sy) != 0 else 1.0)
    else:
        fsy = np.float32(sy) if np.float32(sy) != 0 else np.float32(1.0)
        mult = np.float64((np.float32(sa) * np.float32(sw)) / fsy)
    v = np.clip(np.rint(acc.astype(np.float64) * mult) + zpy, -128, 127).astype(np.int32)
    return v.reshape(-1)[:ny]


@pytest.mark.parametrize("recipe", [0, 1])
def test_qlinear_matmul_bruteforce(recipe):
    """QLinearMatMul (session.tkv:1992-2071) against numpy: random codes and
    zero points, exact half-way products (mult = 1/2 with odd sums), short
    A / B (reads past the end are 0, not (0 - zp)), short Y, sy == 0, k == 0."""
    for case in range(40):
        m, n, k = (int(v) for v in RNG.integers(1, 9, 3))
        if case == 0:
            k = 0
        a = RNG.integers(-128, 128, m * k).astype(np.int32)
        b = RNG.integers(-128, 128, k * n).astype(np.int32)
        if case % 5 == 1 and a.size > 1:
            a = a[:-2]
        if case % 7 == 2 and b.size > 1:
            b = b[:-3]
        zpa, zpw, zpy = (int(v) for v in RNG.integers(-20, 21, 3))
        if case % 3 == 0:
            sa, sw, sy = 0.5, 1.0, 1.0           # every odd sum is a tie
        else:
            sa, sw = (float(np.float32(v)) for v in RNG.uniform(0.001, 0.05, 2))
            sy = 0.0 if case % 11 == 4 else float(np.float32(RNG.uniform(0.05, 2.0)))
        ny = m * n - (1 if case % 4 == 3 else 0)
        got = O.qlinear_matmul(a, sa, zpa, b, sw, zpw, sy, zpy, ny, m, n, k, recipe)
        want = _qlinear_numpy(a, sa, zpa, b, sw, zpw, sy, zpy, ny, m, n, k, recipe)
        assert np.array_equal(got, want), case
    # a planted rounding mistake (half away from zero) is caught by the ties
    acc = np.array([1, 3, 5, -1, -3], np.int64)
    assert not np.array_equal(np.rint(acc * 0.5), np.floor(acc * 0.5 + 0.5))


# ---------------------------------------------------------------------------
# heavier calibrators (engine.tkv:42-197)
# ---------------------------------------------------------------------------

def _calib_data(n, seed):
    x = O.gi_noise(n, seed, 1.0)
    return O.add_outliers(x, 0.01, seed + 1, seed + 2, 20.0) if n > 100 else x


@pytest.mark.parametrize("n,bins,target", [(5000, 2048, 128), (20000, 512, 32), (3000, 64, 8)])
def test_calibrate_kl_closed_form(n, bins, target):
    """At th = target_bins every q equals p (per = 1 and the last block is the
    merged tail itself), so KL = 0 exactly and no later candidate can beat it
    on data whose tail bins differ: thr = target * max|x| / num_bins."""
    x = _calib_data(n, 17)
    am = float(np.max(np.abs(x.astype(np.float64))))
    thr = target * (am / bins)
    p = O.calibrate_kl(x, bins, target)
    assert p.zero_point == 0
    assert p.scale == np.float32(thr / 127.0)
    assert p.min_val == np.float32(-thr) and p.max_val == np.float32(thr)
    assert O.calibrate_kl(np.zeros(7, np.float32)) == O.calibrate_minmax(np.zeros(7, np.float32), 1)


@pytest.mark.parametrize("n", [1, 2, 7, 1000, 50001])
@pytest.mark.parametrize("pct", [99.99, 50.0, 100.0, 0.5])
def test_calibrate_percentile_vs_numpy(n, pct):
    """Clip = sorted |x| at int(min(n - 1, f64(pct) / 100 * n)) (numpy sort);
    asymmetric min / max: data[0] unclipped, the rest clipped (numpy)."""
    x = _calib_data(n, 23)
    ab = np.sort(np.abs(x))
    idx = int(min(n - 1, float(np.float32(pct)) / 100.0 * n))
    clip = max(float(ab[idx]), 1e-8)
    p = O.calibrate_percentile(x, pct, 1)
    assert p.scale == np.float32(clip / 127.0) and p.max_val == np.float32(clip)
    q = O.calibrate_percentile(x, pct, 0)
    c = np.clip(x[1:].astype(np.float64), -clip, clip)
    mn = min(float(x[0]), float(c.min())) if n > 1 else float(x[0])
    mx = max(float(x[0]), float(c.max())) if n > 1 else float(x[0])
    if abs(mx - mn) < 1e-8:
        mx = mn + 1e-8
    assert q.min_val == np.float32(mn) and q.max_val == np.float32(mx)
    assert q.scale == np.float32((mx - mn) / 255.0)
    assert q.zero_point == int(np.clip(np.rint(-mn / ((mx - mn) / 255.0)) - 128, -128, 127))
    for bad in (0.0, -1.0, 100.5):
        with pytest.raises(ValueError):
            O.calibrate_percentile(x, bad)


@pytest.mark.parametrize("n,cands", [(3000, 50), (800, 4), (20000, 17)])
def test_calibrate_mse_argmin_vs_numpy(n, cands):
    """The chosen threshold minimizes the quantization MSE among the
    candidates, recomputed with numpy's vectorized arithmetic (a different
    summation order: agreement holds away from near-ties)."""
    x = _calib_data(n, 31).astype(np.float64)
    am = float(np.max(np.abs(x)))
    mses = []
    for c in range(1, cands + 1):
        thr = am * c / cands
        scale = thr / 127.0
        inv = 1.0 / scale
        q = np.clip(np.rint(np.clip(x, -thr, thr) * inv), -127, 127)
        mses.append(float(np.mean((x - q * scale) ** 2)))
    best = int(np.argmin(mses)) + 1
    srt = sorted(mses)
    assert srt[1] - srt[0] > 1e-9 * srt[0], "test data must not produce a near-tie"
    thr = am * best / cands
    p = O.calibrate_mse(x.astype(np.float32), cands)
    assert p.scale == np.float32(thr / 127.0) and p.max_val == np.float32(thr)


def test_quantize_linear_per_tensor_and_axis():
    x = RNG.normal(0, 3, (2, 3, 4)).astype(np.float32)
    y = O.quantize_linear(x, [0.05], zero_point=3)
    want = np.clip(np.rint(x.astype(np.float64) / np.float64(np.float32(0.05))) + 3, -128, 127)
    assert np.array_equal(y, want.reshape(-1))
    sc = np.array([0.02, 0.1, 1e-13], np.float32)               # last clamps to 1e-12
    y = O.quantize_linear(x, sc, 0, 2, 3, 4).reshape(2, 3, 4)
    s64 = np.maximum(sc.astype(np.float64), 1e-12)
    want = np.clip(np.rint(x.astype(np.float64) / s64[None, :, None]), -128, 127)
    assert np.array_equal(y, want)
    q = RNG.integers(-128, 128, 24).astype(np.int32)
    d = O.dequantize_linear(q, [0.25], 5)
    assert np.array_equal(d, ((q.astype(np.float64) - 5) * 0.25).astype(np.float32))


def test_quantized_gemm_node_dispatch():
    m, n, k = 3, 4, 32
    a = RNG.integers(-127, 128, (m, k)).astype(np.int32)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int32)
    sw = np.full(n, 0.001, np.float32)
    y1 = O.quantized_gemm_node(a, w, None, m, n, k, 0.5, 0.25, sw)
    assert np.array_equal(y1, O.matmul_int8_per_channel(a, w, None, m, n, k, 0.5, sw))
    y2 = O.quantized_gemm_node(a, w, None, m, n, k, 0.5, 0.25, [])
    assert np.array_equal(y2, O.matmul_int8_symmetric(a, w, None, m, n, k, 0.5, 0.25))


# ---------------------------------------------------------------------------
# input generator (gpt2_ref.tkv:1977-1991)
# ---------------------------------------------------------------------------

def test_generator_recurrence_and_moments():
    s, seq = 7, []
    for _ in range(4):
        s = (s * 1103515245 + 12345) % 2 ** 31
        seq.append(s)
    t = 7
    for want in seq:
        t = O.lib().tkvo_lcg31(t)
        assert t == want
    z = O.gi_noise(200000, 0, 1.0)
    assert abs(float(z.mean())) < 0.01 and abs(float(z.std()) - 1.0) < 0.01
    assert np.array_equal(z, O.gi_noise(200000, 0, 1.0))
    x = O.add_outliers(z, 0.001, 3, 4, 20.0)
    assert int(np.sum(x != z)) == 200
