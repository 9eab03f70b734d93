"""How much the compiler typing left unpinned can matter on the benchmark's
own inputs.

Three spots of the reference's arithmetic depend on how tkvc types float
expressions, which only running tkvc-compiled .NET could settle:
  R3   quantize_int8_symmetric's reciprocal 1.0/scale (engine.tkv:219-224):
       f32 (primary) or f64 (alternate);
  R11  matmul_int8_per_channel's epilogue acc * sa * sw[n] + b
       (matmul.tkv:28-29): f64 chain (primary) or f32 chain (alternate);
  QL   QLinearMatMul's multiplier sa * sw / sy (session.tkv:2024-2027): f64
       locals (primary) or an f32 chain (alternate).
The oracle implements both readings of each.  This file counts, on every
BASELINE config's seeded inputs, how many results differ between them:
  * R3: int8 codes that differ (a code moves by 1 only where x * inv lies
    within ~2^-24 relative of a half-integer);
  * R11: the largest |y_primary - y_alternate| / |y|, which stays below the
    north star's 1e-5 relative wherever |y| is not a cancellation of
    acc * s and b, and the abs+rel bound
        |y_p - y_a| <= 2^-21 * (|acc * sa * sw| + |b|)
    everywhere (the f32 chain rounds three times, the f64 chain once);
  * QL: requantized int8 outputs that differ (by exactly 1 where they do).
Run with -s to print the table of counts.

The exact INT32 accumulators come from a float64 matrix product of the
codes: every product is an integer below 2^14 and every partial sum an
integer below 2^53, so BLAS is exact in any order.  The vectorized
epilogues are checked against the oracle's scalar functions on sample rows.
"""
import numpy as np
import pytest

import oracle as O

GPT2 = [("qkv", 2304, 768), ("attn_out", 768, 768), ("mlp_up", 3072, 768),
        ("mlp_down", 768, 3072)]
TABLE = []


def note(row):
    TABLE.append(row)
    print(row, flush=True)


def _r3_diff(x):
    p = O.calibrate_minmax(x, 1)
    q0 = O.quantize_int8_symmetric(x, p.scale, O.PRIMARY)
    q1 = O.quantize_int8_symmetric(x, p.scale, O.ALTERNATE)
    d = q0 != q1
    assert np.all(np.abs(q0[d] - q1[d]) == 1)
    return int(d.sum()), q0, p.scale


def _epilogues(acc, sa, sw, b):
    """Primary (f64 chain) and alternate (f32 chain) epilogues of
    matmul_int8_per_channel on exact accumulators (float64 matrix)."""
    y0 = ((acc * np.float64(sa)) * sw.astype(np.float64)[None, :]
          + b.astype(np.float64)[None, :]).astype(np.float32)
    t = acc.astype(np.float32) * np.float32(sa)
    t = t * sw[None, :]
    y1 = t + b[None, :]
    return y0, y1


def _r11_report(acc, sa, sw, b):
    """(outputs differing, max relative difference where |y| >= 0.1 of the
    terms' magnitude, outputs whose relative difference passes 1e-5 -- all
    cancellations of acc * s against b, held to the abs bound)."""
    y0, y1 = _epilogues(acc, sa, sw, b)
    d = np.abs(y0.astype(np.float64) - y1.astype(np.float64))
    terms = np.abs(acc * np.float64(sa) * sw.astype(np.float64)[None, :]) + \
        np.abs(b.astype(np.float64))[None, :]
    assert np.all(d <= 2.0 ** -21 * terms)
    ay = np.abs(y0.astype(np.float64))
    big = ay >= 0.1 * terms
    rel = float(np.max(d[big] / ay[big])) if big.any() else 0.0
    assert rel <= 1e-5
    over = int(np.sum(d > 1e-5 * ay))
    assert np.all(ay[d > 1e-5 * ay] < 0.1 * terms[d > 1e-5 * ay])
    return int((d > 0).sum()), rel, over


def _check_vs_oracle(xq, wq, b, sa, sw, k, rows):
    """The vectorized epilogues equal the oracle's scalar function (both
    recipes) on a few rows."""
    n = wq.shape[0]
    acc = xq[rows].astype(np.float64) @ wq.astype(np.float64).T
    y0, y1 = _epilogues(acc, sa, sw, b)
    for recipe, want in ((O.PRIMARY, y0), (O.ALTERNATE, y1)):
        got = O.matmul_int8_per_channel(xq[rows].reshape(-1), wq.reshape(-1), b, len(rows), n, k,
                                        sa, sw, recipe=recipe).reshape(len(rows), n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), recipe


def _weights(n, k, seed_w, seed_b):
    w = O.gi_noise(n * k, seed_w, 0.02)
    b = O.gi_noise(n, seed_b, 0.01)
    sw = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, n, k)], np.float32)
    wq = O.quantize_int8_per_channel(w, n, k, sw).reshape(n, k)
    return wq, sw, b


def test_config1_readings():
    m, n, k = 1024, 3072, 768
    x = O.gi_noise(m * k, 0, 1.0)
    diff, xq, sa = _r3_diff(x)
    xq = xq.reshape(m, k)
    wq, sw, b = _weights(n, k, 1, 2)
    _check_vs_oracle(xq, wq, b, sa, sw, k, np.array([0, 511, 1023]))
    acc = xq.astype(np.float64) @ wq.astype(np.float64).T
    nd, rel, over = _r11_report(acc, sa, sw, b)
    note(f"configs[0] 1024x768 -> 3072: R3 codes differing {diff} of {m * k}; "
         f"R11 outputs differing {nd} of {m * n}, max rel {rel:.2e} where |y| >= 0.1 terms; "
         f"{over} cancellation outputs beyond 1e-5 rel, all within 2^-21 terms")


@pytest.mark.parametrize("m", [1024, 8192, 65536])
def test_config2_readings(m):
    x = O.add_outliers(O.gi_noise(m * 768, 0, 1.0), 0.001, 3, 4, 20.0)
    diff, _, _ = _r3_diff(x)
    note(f"configs[1] {m}x768 (+0.1% outliers): R3 codes differing {diff} of {m * 768}")


def test_config3_readings():
    """Layer 0's four linears at M = 8192 (the bench's activations: seed 0
    for K = 768, seed 7 for K = 3072) plus the R3 counts of both activation
    tensors; QLinearMatMul on the same codes."""
    m = 8192
    acts = {}
    for k, seed in ((768, 0), (3072, 7)):
        x = O.gi_noise(m * k, seed, 1.0)
        diff, xq, sa = _r3_diff(x)
        acts[k] = (xq.reshape(m, k), sa)
        note(f"configs[2] activations {m}x{k}: R3 codes differing {diff} of {m * k}")
    ql_total, ql_diff = 0, 0
    for j, (name, n, k) in enumerate(GPT2):
        xq, sa = acts[k]
        wq, sw, b = _weights(n, k, 10 + j + 1, 10 + j + 51)
        if j == 0:
            _check_vs_oracle(xq, wq, b, sa, sw, k, np.array([5, 4000]))
        acc = xq.astype(np.float64) @ wq.astype(np.float64).T
        nd, rel, over = _r11_report(acc, sa, sw, b)
        note(f"configs[2] layer 0 {name} {m}x{k} -> {n}: R11 outputs differing {nd} of {m * n}, "
             f"max rel {rel:.2e} where |y| >= 0.1 terms; {over} cancellation outputs beyond "
             f"1e-5 rel, all within 2^-21 terms")
        # QLinearMatMul on the same codes with a per-tensor weight scale and
        # the output scale of the float result's range: both multipliers
        swt = np.float32(np.max(sw))
        sy = np.float32(np.max(np.abs(acc)) * np.float64(sa) * np.float64(swt) / 127.0)
        m0 = np.float64(sa) * np.float64(swt) / np.float64(sy)
        m1 = np.float64(np.float32(np.float32(sa) * swt) / sy)
        y0 = np.clip(np.rint(acc * m0), -128, 127)
        y1 = np.clip(np.rint(acc * m1), -128, 127)
        d = y0 != y1
        assert np.all(np.abs(y0[d] - y1[d]) == 1)
        if j == 0:
            rows = slice(0, 2)
            for recipe, want in ((O.PRIMARY, y0[rows]), (O.ALTERNATE, y1[rows])):
                got = O.qlinear_matmul(xq[rows].reshape(-1), sa, 0, wq.T.copy().reshape(-1), swt, 0,
                                       sy, 0, 2 * n, 2, n, k, recipe=recipe)
                assert np.array_equal(np.asarray(got).reshape(2, n), want.astype(np.int32)), recipe
        ql_total += m * n
        ql_diff += int(d.sum())
    note(f"configs[2] layer 0, QLinearMatMul mult readings: outputs differing {ql_diff} of {ql_total}")


def test_config5_readings():
    """Decode batches: per-token activation scales (R5, pinned f64) feed the
    per-token form of the R11 epilogue."""
    for (name, n, k) in (("qkv", 2304, 768), ("mlp_up", 3072, 768), ("mlp_down", 768, 3072)):
        wq, sw, b = _weights(n, k, 300, 400)
        worst, nd_tot, over_tot = 0.0, 0, 0
        for m in (1, 4, 16, 32):
            x = O.gi_noise(m * k, 24, 1.0)
            xq, sa = O.quantize_dynamic_int8_rowwise(x, m, k)
            acc = xq.reshape(m, k).astype(np.float64) @ wq.astype(np.float64).T
            y0 = ((acc * sa.astype(np.float64)[:, None]) * sw.astype(np.float64)[None, :]
                  + b.astype(np.float64)[None, :]).astype(np.float32)
            y1 = (acc.astype(np.float32) * sa[:, None]) * sw[None, :] + b[None, :]
            d = np.abs(y0.astype(np.float64) - y1.astype(np.float64))
            terms = np.abs(acc * sa.astype(np.float64)[:, None] * sw.astype(np.float64)[None, :]) \
                + np.abs(b.astype(np.float64))[None, :]
            assert np.all(d <= 2.0 ** -21 * terms)
            ay = np.abs(y0.astype(np.float64))
            big = ay >= 0.1 * terms
            worst = max(worst, float(np.max(d[big] / ay[big])))
            nd_tot += int((d > 0).sum())
            over_tot += int(np.sum(d > 1e-5 * ay))
        assert worst <= 1e-5
        note(f"configs[4] {name} M in 1,4,16,32: R11 (per-token) outputs differing {nd_tot}, "
             f"max rel {worst:.2e} where |y| >= 0.1 terms; {over_tot} cancellation outputs "
             f"beyond 1e-5 rel, all within 2^-21 terms")
