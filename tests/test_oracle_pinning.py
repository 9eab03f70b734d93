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
# FP8 W8A8 linear (R-ext, the scaled extension of matmul.tkv:46-66)
# ---------------------------------------------------------------------------

def _fp8_pack_check(x, codes, s):
    """Independent restatement of one scaled e4m3 pack: the scale is the
    correctly rounded f32 of fl64(max|x| / 240) (Fractions), the codes the
    spec encoder's on numpy's f32 product, and the round trip within half an
    e4m3 step (a full subnormal step in the reference's clamped band)."""
    am = Fraction(float(np.max(np.abs(x.astype(np.float64)))))
    am = max(am, Fraction(1e-8))
    assert s == np.float32(float(am / 240)), (s, float(am))
    inv = np.float32(1.0) / s
    xs = x * inv                                       # numpy f32 multiply (RNE)
    assert np.array_equal(codes + 128, [O.spec_e4m3_encode(float(v)) for v in xs])
    ocp = np.array([_ocp_e4m3_value(int(c)) for c in codes + 128])
    err = np.abs(ocp - xs.astype(np.float64))
    normal = np.abs(xs) >= 2.0 ** -6
    assert np.all(err[normal] <= 2.0 ** -4 * np.abs(xs[normal]))
    assert np.all(err[~normal] <= 2.0 ** -9)
    top = np.argmax(np.abs(x))                         # amax maps to +-240 (code 0x77)
    assert (codes[top] + 128) & 0x7F == 0x77


def test_fp8_act_pack_closed_form():
    x = O.add_outliers(O.gi_noise(6000, 5, 1.0), 0.001, 3, 4, 20.0)
    x[17] = -np.max(np.abs(x)) * 1.5                   # a negative extreme
    codes, s = O.quantize_fp8_e4m3_dynamic_tensor(x)
    _fp8_pack_check(x, codes, s)
    # a tiny-range tensor lands on the 1e-8 scale floor (codes all subnormal or 0)
    z = np.full(64, 3e-9, np.float32)
    codes, s = O.quantize_fp8_e4m3_dynamic_tensor(z)
    assert s == np.float32(1e-8 / 240)
    assert np.array_equal(codes + 128, [O.spec_e4m3_encode(float(v)) for v in z * (np.float32(1) / s)])
    # calibrate_minmax seeds min / max with x[0]: a leading NaN gives a NaN scale
    codes, s = O.quantize_fp8_e4m3_dynamic_tensor(np.array([np.nan, 1.0, -2.0], np.float32))
    assert np.isnan(s)


def test_fp8_weight_pack_per_row():
    rows, cols = 37, 200
    w = O.gi_noise(rows * cols, 9, 0.02).reshape(rows, cols)
    w[3] *= 100.0                                      # rows of very different ranges
    w[5] = 0.0                                         # an all-zero row: scale floor
    codes, sc = O.fp8_weight_pack(w, rows, cols)
    codes = codes.reshape(rows, cols)
    for r in range(rows):
        if r == 5:
            assert sc[r] == np.float32(1e-8 / 240) and np.all(codes[r] == -128)
            continue
        _fp8_pack_check(w[r], codes[r], sc[r])
        c2, s2 = O.quantize_fp8_e4m3_dynamic_tensor(w[r])
        assert s2 == sc[r] and np.array_equal(c2, codes[r])


def _fp8_codes_any(shape):
    codes = [c for c in range(256) if (c & 0x7F) != 0x7F]
    return (RNG.choice(codes, shape) - 128).astype(np.int32)


def test_fp8_scaled_gemm_unit_and_power_of_two_scales():
    """sa = sw = 1 reduces to matmul_fp8_e4m3 (pinned above by Fractions);
    power-of-two scales commute with every rounding, so
    y(sa = 2^ea, sw[n] = 2^eb[n], b) == 2^(ea + eb[n]) * y_unscaled(b * 2^-(ea + eb[n]))
    bit for bit.  A dropped scale, sw indexed by row, or a bias applied
    before the scaling fails it."""
    m, n, k = 6, 9, 96
    a, w = _fp8_codes_any((m, k)), _fp8_codes_any((n, k))
    b = RNG.normal(0, 1, n).astype(np.float32)
    y1 = O.matmul_fp8_e4m3_scaled(a, w, b, m, n, k, np.float32(1), np.ones(n, np.float32))
    assert np.array_equal(y1.view(np.uint32), O.matmul_fp8_e4m3(a, w, b, m, n, k).view(np.uint32))
    ea = -7
    eb = RNG.integers(-12, -3, n)
    sw = (2.0 ** eb).astype(np.float32)
    y = O.matmul_fp8_e4m3_scaled(a, w, b, m, n, k, np.float32(2.0 ** ea), sw).reshape(m, n)
    bs = (b.astype(np.float64) * 2.0 ** -(ea + eb)).astype(np.float32)
    assert np.array_equal(bs.astype(np.float64) * 2.0 ** (ea + eb), b.astype(np.float64))
    yu = O.matmul_fp8_e4m3(a, w, bs, m, n, k).reshape(m, n).astype(np.float64)
    want = (yu * 2.0 ** (ea + eb)[None, :]).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_fp8_scaled_gemm_fraction_bound_and_per_token():
    """General scales: within half an f32 ulp plus two f64 roundings of the
    exact S * sa * sw + b (Fractions); per-token scales index by row."""
    m, n, k = 5, 7, 64
    a, w = _fp8_codes_any((m, k)), _fp8_codes_any((n, k))
    b = RNG.normal(0, 0.01, n).astype(np.float32)
    sa = RNG.uniform(0.001, 0.05, m).astype(np.float32)
    sw = RNG.uniform(1e-4, 3e-4, n).astype(np.float32)
    y = O.matmul_fp8_e4m3_scaled(a, w, b, m, n, k, sa, sw, per_token=True).reshape(m, n)
    t = _dec_table()
    da, dw = t[a + 128], t[w + 128]
    for i in range(m):
        yt = O.matmul_fp8_e4m3_scaled(a[i:i + 1], w, b, 1, n, k, sa[i], sw)
        assert np.array_equal(yt.view(np.uint32), y[i].view(np.uint32))
        for j in range(n):
            s = sum(Fraction(float(p)) for p in da[i] * dw[j])
            ex = s * Fraction(float(sa[i])) * Fraction(float(sw[j])) + Fraction(float(b[j]))
            mag = abs(s * Fraction(float(sa[i])) * Fraction(float(sw[j]))) + abs(Fraction(float(b[j])))
            tol = Fraction(float(np.spacing(np.float32(abs(float(ex)))))) / 2 + mag * Fraction(3, 2 ** 53)
            assert abs(Fraction(float(y[i, j])) - ex) <= tol, (i, j)


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


# ---------------------------------------------------------------------------
# grouped INT4 (int4.tkv) and GGUF block formats (gguf.tkv)
# ---------------------------------------------------------------------------

def _bytes(q):
    """Pack nibble codes q[c] into the reference's bytes: low nibble = even c."""
    q = np.asarray(q, np.int64)
    return ((q[1::2] << 4) | q[0::2]).astype(np.int32)


def test_int4_reference_kat():
    """inference_tests.tkv:634-652 (test_awq_asym_and_fp16): a 1x8 ramp in
    groups of 4 round-trips within 2 * max(scales); permute / inverse
    permute restore the data (nonzero data here, zeros in the reference)."""
    w = np.array([i - 2.0 for i in range(8)], np.float32)
    pk, sc, zp = O.quantize_int4_grouped_asym(w, 1, 8, 4)
    assert pk.size == 4 and sc.size == 2 and zp.size == 2
    y = O.dequantize_int4_grouped_asym(pk, 1, 8, 4, sc, zp)
    assert np.all(np.abs(w - y) < float(sc.max()) * 2.0)
    p = np.arange(1, 7, dtype=np.float32)
    fwd = O.permute_cols(p, 2, 3, [2, 0, 1])
    assert np.array_equal(fwd, np.array([3, 1, 2, 6, 4, 5], np.float32))   # out[r,c] = src[r,perm[c]]
    assert np.array_equal(O.permute_cols(fwd, 2, 3, [2, 0, 1], inverse=True), p)
    with pytest.raises(ValueError):
        O.permute_cols(p, 2, 3, [0, 1])


def test_int4_sym_closed_forms():
    # group max 7 -> scale exactly 1: codes are round-half-even(x) + 8, low nibble first
    g = np.array([7.0, -7.0, 3.5, 2.5, -2.5, -0.5, 0.5, 1.5], np.float32)
    pk, sc = O.quantize_int4_grouped(g, 1, 8, 8)
    assert sc[0] == np.float32(1.0)
    q = np.array([7, -7, 4, 2, -2, 0, 0, 2])
    assert np.array_equal(pk, _bytes(q + 8))
    assert np.array_equal(O.dequantize_int4_grouped(pk, 1, 8, 8, sc), q.astype(np.float32))
    # scale = fl32(am / 7); a flat group floors am at 1e-8 and codes to 8
    _, sc = O.quantize_int4_grouped(np.array([1, 0, 0, 0], np.float32), 1, 4, 4)
    assert sc[0] == np.float32(1.0 / 7.0)
    pk, sc = O.quantize_int4_grouped(np.zeros(4, np.float32), 1, 4, 4)
    assert sc[0] == np.float32(1e-8 / 7.0) and np.all(pk == 0x88)
    # odd group size: pair (c, c + 1) takes the scale of group c // gs.  Element 3
    # (group 1, scale 1) is coded with group 0's scale 0.1: 3 / 0.1 clamps to 7.
    x = np.array([0.7, 0.1, 0.1, 3.0, 7.0, 7.0], np.float32)
    pk, sc = O.quantize_int4_grouped(x, 1, 6, 3)
    assert sc[1] == np.float32(1.0)
    assert np.array_equal(pk, _bytes(np.array([7, 1, 1, 7, 7, 7]) + 8))
    y = O.dequantize_int4_grouped(pk, 1, 6, 3, sc)
    assert y[3] == np.float32(7.0 * float(sc[0]))
    # packed entries past rows * cols / 2 are cleared, as the reference clears the list
    pk, _ = O.quantize_int4_grouped(g, 1, 8, 8, npacked=7)
    assert pk.size == 7 and np.all(pk[4:] == 0)
    with pytest.raises(ValueError):
        O.quantize_int4_grouped(g, 1, 8, 3)


def test_int4_asym_branches():
    # ramp 0 .. 15 s: zp 0 (mn == 0 is not > 0), sc = (mx - mn) / 15 = s, codes = i
    s = 0.25
    pk, sc, zp = O.quantize_int4_grouped_asym((np.arange(16) * s).astype(np.float32), 1, 16, 16)
    assert sc[0] == np.float32(s) and zp[0] == 0
    assert np.array_equal(pk, _bytes(np.arange(16)))
    # all-positive group (int4.tkv:118-137): zp 0 and sc = mx / 15
    pk, sc, zp = O.quantize_int4_grouped_asym(np.array([2, 3, 4, 5], np.float32), 1, 4, 4)
    assert zp[0] == 0 and sc[0] == np.float32(5.0 / 15.0)
    assert np.array_equal(pk, _bytes([6, 9, 12, 15]))
    # all-negative group: zp clamps to 15, sc = -mn / 15
    pk, sc, zp = O.quantize_int4_grouped_asym(np.array([-5, -4, -3, -2], np.float32), 1, 4, 4)
    assert zp[0] == 15 and sc[0] == np.float32(5.0 / 15.0)
    y = O.dequantize_int4_grouped_asym(pk, 1, 4, 4, sc, zp)
    assert np.all(np.abs(y - np.array([-5, -4, -3, -2])) <= float(sc[0]) / 2 + 1e-6)
    # straddling zero: zp = round(-mn / sc) = round(1 / 0.2) = 5
    pk, sc, zp = O.quantize_int4_grouped_asym(np.array([-1, 0, 1, 2], np.float32), 1, 4, 4)
    assert zp[0] == 5 and sc[0] == np.float32(0.2)
    assert np.array_equal(pk, _bytes([0, 5, 10, 15]))
    # flat group: mx = mn + 1e-8, sc floored at 1e-8
    pk, sc, zp = O.quantize_int4_grouped_asym(np.full(4, 3.0, np.float32), 1, 4, 4)
    assert sc[0] == np.float32(max(3.0 / 15.0, 1e-8)) and zp[0] == 0


def test_int4_roundtrip_error_bound():
    """Every element of a group lies within the group's code range, so the
    round trip errs by at most half a step (plus the f32 rounding of the
    stored scale): |dq - x| <= sc / 2 (1 + 2^-18)."""
    rows, cols, gs = 24, 256, 32
    x = RNG.normal(0, 1, rows * cols).astype(np.float32)
    x[::37] *= 30
    x[:gs] = np.abs(x[:gs]) + 0.5       # an all-positive group
    x[gs:2 * gs] = -np.abs(x[gs:2 * gs]) - 0.5   # an all-negative group
    ng = cols // gs
    pk, sc = O.quantize_int4_grouped(x, rows, cols, gs)
    y = O.dequantize_int4_grouped(pk, rows, cols, gs, sc)
    step = np.repeat(sc.astype(np.float64), gs)
    assert np.all(np.abs(y.astype(np.float64) - x) <= step / 2 * (1 + 2.0 ** -18))
    pk, sc, zp = O.quantize_int4_grouped_asym(x, rows, cols, gs)
    assert np.all((zp >= 0) & (zp <= 15)) and sc.size == rows * ng
    y = O.dequantize_int4_grouped_asym(pk, rows, cols, gs, sc, zp)
    step = np.repeat(sc.astype(np.float64), gs)
    # zp == 15 reached by rounding (-mn / sc in [14.5, 15)) with mx > 0 takes
    # sc = -mn / 15, whose range [mn, 0] clips mx <= sc0 / 2 <= (15 / 29) sc
    err = np.abs(y.astype(np.float64) - x)
    assert np.all(err <= step * 15 / 29 * (1 + 2.0 ** -18) + 1e-7)
    g15 = np.repeat(zp == 15, gs)
    assert np.all(err[~g15] <= step[~g15] / 2 * (1 + 2.0 ** -18) + 1e-7)


def _int4_dense(packed, scales, n, k, gs):
    """Independent decode: nibble kk of row n is byte kk // 2, low nibble first,
    scaled by the group of kk itself (matmul indexes per element)."""
    b = np.asarray(packed, np.int64).reshape(n, k // 2)
    nib = np.empty((n, k), np.int64)
    nib[:, 0::2], nib[:, 1::2] = b & 15, (b >> 4) & 15
    sc = np.asarray(scales, np.float64).reshape(n, k // gs)
    return (nib - 8) * np.repeat(sc, gs, axis=1)


def test_int4_matmul_exact_dyadic():
    """Dyadic activations and power-of-two scales keep every partial sum
    exact, so any summation order gives the reference's value: bit-exact
    against an independent dense decode + f64 matmul."""
    m, n, k, gs = 6, 9, 96, 32
    a = (RNG.integers(-64, 64, m * k) / 16.0).astype(np.float32)
    pk = RNG.integers(0, 256, n * k // 2).astype(np.int32)
    sc = (2.0 ** -RNG.integers(1, 6, n * k // gs)).astype(np.float32)
    b = (RNG.integers(-8, 8, n) / 8.0).astype(np.float32)
    w = _int4_dense(pk, sc, n, k, gs)
    want = (a.astype(np.float64).reshape(m, k) @ w.T + b.astype(np.float64)).astype(np.float32)
    assert np.array_equal(O.matmul_int4_grouped(a, pk, b, m, n, k, gs, sc), want.reshape(-1))
    want0 = (a.astype(np.float64).reshape(m, k) @ w.T).astype(np.float32)
    assert np.array_equal(O.matmul_int4_grouped(a, pk, None, m, n, k, gs, sc), want0.reshape(-1))
    with pytest.raises(ValueError):
        O.matmul_int4_grouped(a, pk, b, m, n, k, gs, sc[:-1])


def test_int4_matmul_general_and_ordered():
    """General data: within the f64 reordering bound of the dense product.
    The act-order form is the plain form on column-permuted activations, bit
    for bit (same products in the same order)."""
    m, n, k, gs = 7, 11, 128, 64
    a = RNG.normal(0, 1, m * k).astype(np.float32)
    w = RNG.normal(0, 0.05, n * k).astype(np.float32)
    pk, sc = O.quantize_int4_grouped(w, n, k, gs)
    b = RNG.normal(0, 0.1, n).astype(np.float32)
    y = O.matmul_int4_grouped(a, pk, b, m, n, k, gs, sc).astype(np.float64)
    wd = _int4_dense(pk, sc, n, k, gs)
    A = a.astype(np.float64).reshape(m, k)
    ref = (A @ wd.T + b.astype(np.float64)).reshape(-1)
    bound = k * 2.0 ** -52 * (np.abs(A) @ np.abs(wd).T).reshape(-1) + np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(y - ref) <= bound)
    perm = RNG.permutation(k)
    yo = O.matmul_int4_grouped(a, pk, b, m, n, k, gs, sc, perm=perm)
    ap = O.permute_cols(a, m, k, perm)
    assert np.array_equal(yo, O.matmul_int4_grouped(ap, pk, b, m, n, k, gs, sc))


def test_f16_decoder_all_codes():
    """Every binary16 code against numpy's conversion (NaN as NaN)."""
    h = np.arange(65536, dtype=np.int64)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_gguf_block_known_answers():
    q = (np.arange(32) * 8 - 128).astype(np.int8)
    blk8 = np.concatenate([np.array([0x00, 0x38], np.uint8), q.view(np.uint8)])  # d = 0.5
    neg8 = np.concatenate([np.array([0x00, 0xC0], np.uint8), q.view(np.uint8)])  # d = -2
    raw = np.concatenate([blk8, neg8])
    y = O.dequantize_gguf(raw, 70, O.GGUF_Q8_0)                    # 2 blocks + 6 tail zeros
    assert np.array_equal(y[:32], 0.5 * q.astype(np.float32))
    assert np.array_equal(y[32:64], -2.0 * q.astype(np.float32))
    assert np.all(y[64:] == 0)
    lo, hi = np.arange(16), (np.arange(16) * 7) % 16
    qs = (hi << 4 | lo).astype(np.uint8)
    y = O.dequantize_gguf(np.concatenate([np.array([0x00, 0x40], np.uint8), qs]), 32, O.GGUF_Q4_0)
    assert np.array_equal(y[:16], 2.0 * (lo - 8)) and np.array_equal(y[16:], 2.0 * (hi - 8))
    y = O.dequantize_gguf(np.concatenate([np.array([0x00, 0x34, 0x00, 0x3E], np.uint8), qs]), 32,
                          O.GGUF_Q4_1)                             # d = 0.25, m = 1.5
    assert np.array_equal(y[:16], 0.25 * lo - 1.5) and np.array_equal(y[16:], 0.25 * hi - 1.5)
    # a subnormal half scale: d = 2^-24 (code 0x0001)
    y = O.dequantize_gguf(np.concatenate([np.array([0x01, 0x00], np.uint8), q.view(np.uint8)]), 32,
                          O.GGUF_Q8_0)
    assert np.array_equal(y, (q.astype(np.float64) * 2.0 ** -24).astype(np.float32))
    with pytest.raises(ValueError):
        O.dequantize_gguf(raw[:40], 64, O.GGUF_Q8_0)


# ---------------------------------------------------------------------------
# Q8_0 weights on int8 activation codes (an extension: the reference decodes
# Q8_0 blocks to f32, gguf.tkv:284-290, and has no quantized GEMM for them)
# ---------------------------------------------------------------------------

def q8_0_blocks(rows, kb, d_codes, q):
    """Raw Q8_0 bytes of rows x kb blocks: f16 scale codes d_codes [rows, kb]
    and int8 codes q [rows, kb * 32]."""
    raw = np.zeros((rows, kb, 34), np.uint8)
    raw[:, :, 0] = d_codes & 255
    raw[:, :, 1] = (d_codes >> 8) & 255
    raw[:, :, 2:] = np.asarray(q, np.int8).reshape(rows, kb, 32).view(np.uint8)
    return raw.reshape(-1)


def _round_f32(x: Fraction) -> Fraction:
    """x rounded to the nearest f32 (ties to even), finite range."""
    if x == 0:
        return Fraction(0)
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** (max(e, -126) - 23)
    q = a / ulp
    whole = q.numerator // q.denominator
    rest = q - whole
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and whole % 2 == 1):
        whole += 1
    assert whole * ulp < Fraction(2) ** 128
    return (whole * ulp) if x > 0 else -(whole * ulp)


def test_q8_0_matmul_exact_on_dyadic_inputs():
    """Power-of-two group scales and small codes keep every step of the fma
    chain exact, so y is the exact product of the reference decoder's weights
    (dequantize_gguf, gguf.tkv:284-290) with the activation codes, scaled and
    biased once in f64: pins the block layout, the row / column roles, the
    per-tensor and per-token scale and the bias against numpy f64 matmul."""
    m, n, k = 7, 9, 256
    kb = k // 32
    e = RNG.integers(-4, 1, (n, kb))
    d_codes = (RNG.integers(0, 2, (n, kb)) << 15) | ((e + 15) << 10)    # +-2^e
    q = RNG.integers(-8, 9, (n, k)).astype(np.int8)
    raw = q8_0_blocks(n, kb, d_codes, q)
    a = RNG.integers(-8, 9, (m, k)).astype(np.int32)
    w = O.dequantize_gguf(raw, n * k, O.GGUF_Q8_0).reshape(n, k).astype(np.float64)
    exact = a.astype(np.float64) @ w.T       # multiples of 2^-4 below 2^14: exact
    bias = RNG.standard_normal(n).astype(np.float32)
    for sa in (np.float32(0.0123), (RNG.random(m) + 0.01).astype(np.float32)):
        s = np.asarray(sa, np.float64).reshape(-1, 1)
        for b in (bias, None):
            want = (exact * s + (0.0 if b is None else b.astype(np.float64))).astype(np.float32)
            got = O.matmul_q8_0(a, raw, sa, m, n, k, b)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError):
        O.matmul_q8_0(a[:, :200], raw, 1.0, m, n, 200)                 # k % 32 != 0
    with pytest.raises(ValueError):
        O.matmul_q8_0(a, raw[:-1], 1.0, m, n, k)                       # raw too short


def test_q8_0_matmul_rounds_once_per_group():
    """General scales and full-range codes: the oracle equals an exact-rational
    emulation of the stated chain (each group's fma rounded once to f32, in
    group order), and on these inputs a chain that rounds the product before
    the add differs from it, so the check tells the two apart."""
    m, n, k = 3, 5, 384
    kb = k // 32
    d_codes = RNG.integers(0x0400, 0x7C00, (n, kb)) | (RNG.integers(0, 2, (n, kb)) << 15)
    q = RNG.integers(-128, 128, (n, k)).astype(np.int8)
    a = RNG.integers(-127, 128, (m, k)).astype(np.int64)
    raw = q8_0_blocks(n, kb, d_codes, q)
    d = d_codes.astype(np.uint16).view(np.float16).astype(np.float64)
    sa = np.float32(0.037)
    got = O.matmul_q8_0(a, raw, sa, m, n, k)
    differs = 0
    for i in range(m):
        for j in range(n):
            fused, split = Fraction(0), Fraction(0)
            for g in range(kb):
                dot = int(a[i, 32 * g:32 * g + 32] @ q[j, 32 * g:32 * g + 32].astype(np.int64))
                dg = Fraction(float(d[j, g]))
                fused = _round_f32(fused + dot * dg)
                split = _round_f32(split + _round_f32(dot * dg))
            differs += fused != split
            want = np.float32(float(fused) * float(sa) + 0.0)
            assert got[i, j].view(np.uint32) == want.view(np.uint32), (i, j)
    assert differs > 0


def test_q8_0_matmul_within_stated_bound_of_float_product():
    """Against the reference's own semantics -- decode the blocks to f32, then
    multiply the float activation -- the per-token int8 codes of x
    (quantize_dynamic_int8_rowwise, engine.tkv:266-285) cost at most
    (sa / 2) sum_k |w[n, k]| per output (plus 128 2^-24 sa sum_k |w|: the
    codes come from the unrounded f64 scale, sa is its f32 rounding), and the
    f32 chain one rounding per group:
    |y - x w^T| <= (sa / 2 + 2^-17 sa) sum_k |w| + kb 2^-24 sum_g |d dot_g| sa + 2^-24 |y|."""
    m, n, k = 6, 11, 512
    kb = k // 32
    d_codes = RNG.integers(0x1C00, 0x2800, (n, kb))                   # 2^-8 .. 2^-5
    q = RNG.integers(-128, 128, (n, k)).astype(np.int8)
    raw = q8_0_blocks(n, kb, d_codes, q)
    x = RNG.standard_normal((m, k)).astype(np.float32)
    codes, sa = O.quantize_dynamic_int8_rowwise(x.reshape(-1), m, k)
    codes = np.asarray(codes, np.int64).reshape(m, k)
    sa = np.asarray(sa, np.float32)
    y = O.matmul_q8_0(codes, raw, sa, m, n, k).astype(np.float64)
    w = O.dequantize_gguf(raw, n * k, O.GGUF_Q8_0).reshape(n, k).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    d = d_codes.astype(np.uint16).view(np.float16).astype(np.float64)
    dots = np.einsum("mgk,ngk->mng", codes.reshape(m, kb, 32), q.astype(np.int64).reshape(n, kb, 32))
    chain = kb * 2.0 ** -24 * np.abs(dots * d[None]).sum(axis=2) * sa[:, None]
    bound = (sa[:, None] / 2 + 2.0 ** -17 * sa[:, None]) * np.abs(w).sum(axis=1)[None] + chain \
        + 2.0 ** -24 * np.abs(y)
    assert np.all(np.abs(y - ref) <= bound)
    # the activation term dominates: the bound is not vacuous
    assert np.abs(y - ref).max() > 0.01 * bound.max()
