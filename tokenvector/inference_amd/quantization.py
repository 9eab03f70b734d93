"""Host-side mirror of the reference's PTQ API, running on libtkv_hip.

Same function names, argument order, in-place ``dst`` semantics, return
value (0) and ValueError cases as the .tkv sources:

    tv/quantization/engine.tkv   calibrate_minmax, calibrate_per_channel_minmax,
                                 quantize_/dequantize_int8_symmetric,
                                 quantize_/dequantize_int8_per_channel,
                                 quantize_dynamic_int8_rowwise
    tv/quantization/matmul.tkv   matmul_int8_symmetric, matmul_int8_per_channel,
                                 matmul_fp8_e4m3, quantize_fp8_e4m3,
                                 dequantize_fp8_e4m3

Code lists (``list[i32]`` in the reference) are int32 numpy arrays; float
lists are float32 arrays.  Every call goes through the C ABI to the GPU;
there is no CPU fallback (a missing library or device raises).
"""
from __future__ import annotations

import ctypes as C
from typing import List, NamedTuple

import numpy as np

from . import _lib

PRIMARY = 0
ALTERNATE = 1


class QuantParams(NamedTuple):
    """QuantParams record (tv/quantization/types.tkv:17-27)."""
    scale: np.float32
    zero_point: int
    min_val: np.float32
    max_val: np.float32


def _f32_in(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))


def _i32_in(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32).reshape(-1))


def _out(arr: np.ndarray, dtype) -> np.ndarray:
    if not isinstance(arr, np.ndarray) or arr.dtype != dtype or not arr.flags["C_CONTIGUOUS"]:
        raise TypeError(f"destination must be a contiguous {np.dtype(dtype).name} ndarray")
    return arr.reshape(-1)


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _bias(pbias):
    if pbias is None:
        return np.zeros(1, dtype=np.float32), 0
    b = _f32_in(pbias)
    return (b if b.size else np.zeros(1, dtype=np.float32)), b.size


# ---- engine.tkv ------------------------------------------------------------

def calibrate_minmax(data, symmetric: int = 1) -> QuantParams:
    """engine.tkv:13-36 -- absmax (symmetric) or min/max (asymmetric) scale."""
    x = _f32_in(data)
    s, mn, mx = C.c_float(), C.c_float(), C.c_float()
    zp = C.c_int64()
    _lib.check(_lib.lib().tkv_hip_calibrate_minmax(_p(x), x.size, int(symmetric), C.byref(s),
                                                   C.byref(zp), C.byref(mn), C.byref(mx)))
    return QuantParams(np.float32(s.value), int(zp.value), np.float32(mn.value), np.float32(mx.value))


def _calib_call(name, x, *args) -> QuantParams:
    s, mn, mx = C.c_float(), C.c_float(), C.c_float()
    zp = C.c_int64()
    rc = getattr(_lib.lib(), name)(_p(x), x.size, *args, C.byref(s), C.byref(zp), C.byref(mn),
                                   C.byref(mx))
    _lib.check(rc)
    return QuantParams(np.float32(s.value), int(zp.value), np.float32(mn.value), np.float32(mx.value))


def calibrate_kl(data, num_bins: int = 2048, target_bins: int = 128) -> QuantParams:
    """engine.tkv:42-123 -- TensorRT-style KL calibration of |x|'s histogram."""
    return _calib_call("tkv_hip_calibrate_kl", _f32_in(data), int(num_bins), int(target_bins))


def calibrate_percentile(data, percentile: float = 99.99, symmetric: int = 1) -> QuantParams:
    """engine.tkv:126-162 -- clip at the percentile of |x|; ValueError outside (0, 100]."""
    x = _f32_in(data)
    if x.size and not (0.0 < np.float32(percentile) <= 100.0):
        raise ValueError("percentile must be in (0, 100]")
    return _calib_call("tkv_hip_calibrate_percentile", x, float(np.float32(percentile)),
                       int(symmetric))


def calibrate_mse(data, num_candidates: int = 50) -> QuantParams:
    """engine.tkv:165-197 -- grid search of symmetric thresholds minimizing the MSE."""
    return _calib_call("tkv_hip_calibrate_mse", _f32_in(data), int(num_candidates))


def calibrate_per_channel_minmax(data, rows: int, cols: int, symmetric: int = 1) -> List[QuantParams]:
    """engine.tkv:202-213 -- calibrate_minmax per row of a [rows, cols] matrix."""
    x = _f32_in(data)
    r = max(int(rows), 0)
    sc = np.zeros(max(r, 1), np.float32)
    zp = np.zeros(max(r, 1), np.int64)
    mn = np.zeros(max(r, 1), np.float32)
    mx = np.zeros(max(r, 1), np.float32)
    _lib.check(_lib.lib().tkv_hip_calibrate_per_channel_minmax(
        _p(x), x.size, int(rows), int(cols), int(symmetric), _p(sc), _p(zp), _p(mn), _p(mx)))
    return [QuantParams(sc[i], int(zp[i]), mn[i], mx[i]) for i in range(r)]


def quantize_int8_symmetric(src, dst: np.ndarray, scale, recipe: int = PRIMARY) -> int:
    """engine.tkv:216-226 -- dst[i] = clamp(round(src[i] / scale), +-127)."""
    x = _f32_in(src)
    d = _out(dst, np.int32)
    return _lib.check(_lib.lib().tkv_hip_quantize_int8_symmetric_recipe(
        _p(x), x.size, _p(d), d.size, float(np.float32(scale)), int(recipe)))


def dequantize_int8_symmetric(src, dst: np.ndarray, scale) -> int:
    """engine.tkv:229-234 -- dst[i] = src[i] * scale."""
    q = _i32_in(src)
    d = _out(dst, np.float32)
    return _lib.check(_lib.lib().tkv_hip_dequantize_int8_symmetric(
        _p(q), q.size, _p(d), d.size, float(np.float32(scale))))


def quantize_int8_per_channel(src, dst: np.ndarray, rows: int, cols: int, scales) -> int:
    """engine.tkv:237-250 -- one scale per row."""
    x = _f32_in(src)
    d = _out(dst, np.int32)
    s = _f32_in(scales)
    return _lib.check(_lib.lib().tkv_hip_quantize_int8_per_channel(
        _p(x), x.size, _p(d), d.size, int(rows), int(cols), _p(s), s.size))


def dequantize_int8_per_channel(src, dst: np.ndarray, rows: int, cols: int, scales) -> int:
    """engine.tkv:253-262"""
    q = _i32_in(src)
    d = _out(dst, np.float32)
    s = _f32_in(scales)
    return _lib.check(_lib.lib().tkv_hip_dequantize_int8_per_channel(
        _p(q), q.size, _p(d), d.size, int(rows), int(cols), _p(s), s.size))


def quantize_dynamic_int8_rowwise(src, dst: np.ndarray, rows: int, cols: int,
                                  scales_out: np.ndarray) -> int:
    """engine.tkv:266-285 -- per-row absmax scale derived on the fly."""
    x = _f32_in(src)
    d = _out(dst, np.int32)
    so = _out(scales_out, np.float32)
    return _lib.check(_lib.lib().tkv_hip_quantize_dynamic_int8_rowwise(
        _p(x), x.size, _p(d), d.size, int(rows), int(cols), _p(so), so.size))


# ---- matmul.tkv ------------------------------------------------------------

def _gemm_sizes(pa, pw, py, m, n, k):
    a, w = _i32_in(pa), _i32_in(pw)
    y = _out(py, np.float32)
    m, n, k = int(m), int(n), int(k)
    # The reference indexes pa[mm*k+kk], pw[nn*k+kk], py[mm*n+nn]: short
    # lists raise there (IndexError), before any arithmetic.
    if a.size < m * k or w.size < n * k or y.size < m * n:
        raise IndexError("operand shorter than m*k / n*k / m*n")
    return a, w, y, m, n, k


def matmul_int8_symmetric(pa, pw, pbias, py: np.ndarray, m, n, k, scale_a, scale_w) -> int:
    """matmul.tkv:4-15 -- y = acc * (scale_a * scale_w) + bias."""
    a, w, y, m, n, k = _gemm_sizes(pa, pw, py, m, n, k)
    b, nb = _bias(pbias)
    return _lib.check(_lib.lib().tkv_hip_matmul_int8_symmetric(
        _p(a), _p(w), _p(b), nb, _p(y), m, n, k, float(np.float32(scale_a)),
        float(np.float32(scale_w))))


def matmul_int8_per_channel(pa, pw, pbias, py: np.ndarray, m, n, k, scale_a, scales_w) -> int:
    """matmul.tkv:17-29 -- y = acc * scale_a * scales_w[n] + bias[n]."""
    s = _f32_in(scales_w)
    if s.size < int(n):
        raise ValueError("scales_w smaller than N")
    a, w, y, m, n, k = _gemm_sizes(pa, pw, py, m, n, k)
    b, nb = _bias(pbias)
    return _lib.check(_lib.lib().tkv_hip_matmul_int8_per_channel(
        _p(a), _p(w), _p(b), nb, _p(y), m, n, k, float(np.float32(scale_a)), _p(s), s.size))


def matmul_int8_recipe(pa, pw, pbias, py, m, n, k, scale_a, scale_w, scales_w, recipe) -> int:
    """Either INT8 GEMM with the epilogue recipe selectable (unpinned typing)."""
    a, w, y, m, n, k = _gemm_sizes(pa, pw, py, m, n, k)
    b, nb = _bias(pbias)
    s = _f32_in(scales_w if scales_w is not None else [])
    sp = s if s.size else np.zeros(1, np.float32)
    return _lib.check(_lib.lib().tkv_hip_matmul_int8_recipe(
        _p(a), _p(w), _p(b), nb, _p(y), m, n, k, float(np.float32(scale_a)),
        float(np.float32(scale_w)), _p(sp), s.size, int(recipe)))


def matmul_int8_accum(pa, pw, m, n, k) -> np.ndarray:
    """INT32 accumulators of the INT8 GEMM (_dot_int8 per output, matmul.tkv:116-127)."""
    a, w = _i32_in(pa), _i32_in(pw)
    acc = np.zeros(int(m) * int(n), np.int32)
    _lib.check(_lib.lib().tkv_hip_matmul_int8_accum(_p(a), _p(w), _p(acc), int(m), int(n), int(k)))
    return acc


def quantize_fp8_e4m3(src, dst: np.ndarray) -> int:
    """matmul.tkv:60-66 -- dst[i] = e4m3 code - 128."""
    x = _f32_in(src)
    d = _out(dst, np.int32)
    return _lib.check(_lib.lib().tkv_hip_quantize_fp8_e4m3(_p(x), x.size, _p(d), d.size))


def dequantize_fp8_e4m3(src, dst: np.ndarray) -> int:
    """matmul.tkv:68-73"""
    q = _i32_in(src)
    d = _out(dst, np.float32)
    return _lib.check(_lib.lib().tkv_hip_dequantize_fp8_e4m3(_p(q), q.size, _p(d), d.size))


def matmul_fp8_e4m3(pa, pw, pbias, py: np.ndarray, m, n, k) -> int:
    """matmul.tkv:46-58 -- y = sum_k dec(a) dec(w) + bias (f32 accumulate here)."""
    a, w, y, m, n, k = _gemm_sizes(pa, pw, py, m, n, k)
    b, nb = _bias(pbias)
    return _lib.check(_lib.lib().tkv_hip_matmul_fp8_e4m3(_p(a), _p(w), _p(b), nb, _p(y), m, n, k))
