"""CPU oracle for the PTQ path -- TEST INFRASTRUCTURE ONLY.

numpy wrappers over ``libtkv_oracle.so`` (the C restatement in
``tkv_oracle.c``).  Only tests, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the timed CPU baseline -- never as the product path.

Each wrapper restates the reference function named in its docstring
(paths relative to the reference checkout).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import NamedTuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libtkv_oracle.so")

PRIMARY = 0
ALTERNATE = 1


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class _QP(C.Structure):
    _fields_ = [("scale", C.c_float), ("zero_point", C.c_int64),
                ("min_val", C.c_float), ("max_val", C.c_float)]


class QuantParams(NamedTuple):
    """QuantParams record (tv/quantization/types.tkv:17-27)."""
    scale: float
    zero_point: int
    min_val: float
    max_val: float

    @staticmethod
    def _from(qp: _QP) -> "QuantParams":
        return QuantParams(np.float32(qp.scale), int(qp.zero_point),
                           np.float32(qp.min_val), np.float32(qp.max_val))


P = C.c_void_p
I64 = C.c_int64
I32 = C.c_int32
F32 = C.c_float
F64 = C.c_double


def _declare(L: C.CDLL) -> None:
    sig = {
        "tkvo_f64_to_f32_bits": (I64, [F64]),
        "tkvo_f32_bits_to_f64": (F64, [I64]),
        "tkvo_rne_rshift": (I64, [I64, I64]),
        "tkvo_fp8_e4m3_encode": (I64, [F32]),
        "tkvo_fp8_e4m3_decode": (F32, [I64]),
        "tkvo_fp8_e5m2_encode": (I64, [F32]),
        "tkvo_fp8_e5m2_decode": (F32, [I64]),
        "tkvo_quant_identity": (_QP, []),
        "tkvo_calibrate_minmax": (_QP, [P, I64, I32]),
        "tkvo_calibrate_kl": (_QP, [P, I64, I64, I64]),
        "tkvo_calibrate_percentile": (_QP, [P, I64, F32, I32, P]),
        "tkvo_calibrate_mse": (_QP, [P, I64, I64]),
        "tkvo_calibrate_per_channel_minmax": (I32, [P, I64, I64, I64, I32, P]),
        "tkvo_quantize_int8_symmetric": (I32, [P, I64, P, F32, I32]),
        "tkvo_dequantize_int8_symmetric": (I32, [P, I64, P, F32]),
        "tkvo_quantize_int8_per_channel": (I32, [P, P, I64, I64, P]),
        "tkvo_dequantize_int8_per_channel": (I32, [P, P, I64, I64, P]),
        "tkvo_quantize_dynamic_int8_rowwise": (I32, [P, P, I64, I64, P]),
        "tkvo_dot_int8": (I64, [P, I64, P, I64, I64]),
        "tkvo_matmul_int8_symmetric": (I32, [P, P, P, I64, P, I64, I64, I64, F32, F32, I32]),
        "tkvo_matmul_int8_per_channel": (I32, [P, P, P, I64, P, I64, I64, I64, F32, P, I64, I32]),
        "tkvo_matmul_int8_per_channel_mt": (I32, [P, P, P, I64, P, I64, I64, I64, F32, P, I64, I32]),
        "tkvo_matmul_int8_accum": (I32, [P, P, P, I64, I64, I64]),
        "tkvo_quantize_fp8_e4m3": (I32, [P, I64, P]),
        "tkvo_dequantize_fp8_e4m3": (I32, [P, I64, P]),
        "tkvo_matmul_fp8_e4m3": (I32, [P, P, P, I64, P, I64, I64, I64]),
        "tkvo_matmul_fp8_e4m3_exact": (I32, [P, P, P, P, I64, I64, I64]),
        "tkvo_quantize_fp8_e4m3_dynamic_tensor": (I32, [P, I64, P, P]),
        "tkvo_fp8_weight_pack": (I32, [P, I64, I64, P, P]),
        "tkvo_matmul_fp8_e4m3_scaled": (I32, [P, P, P, I64, P, I64, I64, I64, P, I64, P]),
        "tkvo_matmul_integer": (I32, [P, I64, P, I64, P, I64, I64, I64, I64]),
        "tkvo_qlinear_matmul": (I32, [P, I64, F32, I64, P, I64, F32, I64, F32, I64, P, I64,
                                      I64, I64, I64, I32]),
        "tkvo_quantize_linear": (I32, [P, I64, P, I64, I64, I64, I64, I64, P]),
        "tkvo_dequantize_linear": (I32, [P, I64, P, I64, I64, I64, I64, I64, P]),
        "tkvo_dynamic_quantize_linear": (I32, [P, I64, P, P, P]),
        "tkvo_quantized_gemm_node": (I32, [P, P, P, I64, P, I64, I64, I64, F32, F32, P, I64, I32]),
        "tkvo_quantize_int4_grouped": (I32, [P, I64, I64, I64, I64, P, I64, P]),
        "tkvo_dequantize_int4_grouped": (I32, [P, I64, P, I64, I64, I64, I64, P, I64]),
        "tkvo_quantize_int4_grouped_asym": (I32, [P, I64, I64, I64, I64, P, I64, P, P]),
        "tkvo_dequantize_int4_grouped_asym": (I32, [P, I64, P, I64, I64, I64, I64, P, P, I64]),
        "tkvo_permute_cols": (I32, [P, I64, I64, P, I64, I32, P]),
        "tkvo_matmul_int4_grouped": (I32, [P, P, P, I64, P, I64, I64, I64, I64, P, I64, P]),
        "tkvo_f16_to_f32": (F32, [I64]),
        "tkvo_dequantize_gguf": (I32, [P, I64, I64, I32, P]),
        "tkvo_matmul_q8_0": (I32, [P, P, I64, P, I64, P, I64, P, I64, I64, I64]),
        "tkvo_lcg31": (I64, [I64]),
        "tkvo_gi_noise": (None, [P, I64, I64, F64]),
        "tkvo_add_outliers": (None, [P, I64, I64, I64, I64, F64]),
        "tkvo_pin_e4m3_spec_encode": (I64, [F32]),
        "tkvo_fp8_e4m3_encode_bits": (I32, [P, I64, P, I32]),
        "tkvo_pin_e4m3_exhaustive": (I64, [I32, I32, I32, C.POINTER(C.c_uint32)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def _i32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.int32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---- generator (tv/training/gpt2_ref.tkv:1977-1991) ----------------------

def gi_noise(n: int, seed: int, sigma: float) -> np.ndarray:
    out = np.empty(int(n), dtype=np.float32)
    lib().tkvo_gi_noise(_p(out), int(n), int(seed), float(sigma))
    return out


def add_outliers(x: np.ndarray, frac: float, seed: int, seed2: int, sigma: float) -> np.ndarray:
    x = _f32(x).copy()
    n_out = int(round(x.size * frac))
    lib().tkvo_add_outliers(_p(x), x.size, n_out, int(seed), int(seed2), float(sigma))
    return x


# ---- f32_bits.tkv / types.tkv ---------------------------------------------

def f64_to_f32_bits(x: float) -> int:
    return int(lib().tkvo_f64_to_f32_bits(float(x)))


def f32_bits_to_f64(b: int) -> float:
    return float(lib().tkvo_f32_bits_to_f64(int(b)))


def rne_rshift(v: int, s: int) -> int:
    return int(lib().tkvo_rne_rshift(int(v), int(s)))


def fp8_e4m3_encode(x: float) -> int:
    return int(lib().tkvo_fp8_e4m3_encode(float(np.float32(x))))


def fp8_e4m3_decode(v: int) -> np.float32:
    return np.float32(lib().tkvo_fp8_e4m3_decode(int(v)))


def fp8_e5m2_encode(x: float) -> int:
    return int(lib().tkvo_fp8_e5m2_encode(float(np.float32(x))))


def fp8_e5m2_decode(v: int) -> np.float32:
    return np.float32(lib().tkvo_fp8_e5m2_decode(int(v)))


def host_threads() -> int:
    """Worker count for threaded oracle helpers: the host's cores, at most 16
    (the CPU share of one GPU on the MI355X boxes)."""
    return max(1, min(16, os.cpu_count() or 1))


def fp8_encode_bits(bits: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """fp8_e4m3_encode of every f32 bit pattern in `bits` (uint32)."""
    b = np.ascontiguousarray(bits, dtype=np.uint32)
    out = np.empty(b.size, np.uint8)
    lib().tkvo_fp8_e4m3_encode_bits(_p(b), b.size, _p(out), int(nthreads or host_threads()))
    return out


def spec_e4m3_encode(x: float) -> int:
    return int(lib().tkvo_pin_e4m3_spec_encode(float(np.float32(x))))


def e4m3_exhaustive(elo: int, ehi: int, nthreads: int = 0):
    bad = C.c_uint32(0)
    n = lib().tkvo_pin_e4m3_exhaustive(int(elo), int(ehi), int(nthreads), C.byref(bad))
    return int(n), int(bad.value)


# ---- engine.tkv ------------------------------------------------------------

def quant_identity() -> QuantParams:
    return QuantParams._from(lib().tkvo_quant_identity())


def calibrate_minmax(data, symmetric: int = 1) -> QuantParams:
    x = _f32(data)
    return QuantParams._from(lib().tkvo_calibrate_minmax(_p(x), x.size, int(symmetric)))


def calibrate_kl(data, num_bins: int = 2048, target_bins: int = 128) -> QuantParams:
    x = _f32(data)
    return QuantParams._from(lib().tkvo_calibrate_kl(_p(x), x.size, int(num_bins),
                                                     int(target_bins)))


def calibrate_percentile(data, percentile: float = 99.99, symmetric: int = 1) -> QuantParams:
    x = _f32(data)
    err = C.c_int32(0)
    r = lib().tkvo_calibrate_percentile(_p(x), x.size, float(np.float32(percentile)),
                                        int(symmetric), C.byref(err))
    if err.value:
        raise ValueError("percentile must be in (0, 100]")
    return QuantParams._from(r)


def calibrate_mse(data, num_candidates: int = 50) -> QuantParams:
    x = _f32(data)
    return QuantParams._from(lib().tkvo_calibrate_mse(_p(x), x.size, int(num_candidates)))


def calibrate_per_channel_minmax(data, rows: int, cols: int, symmetric: int = 1):
    x = _f32(data)
    out = (_QP * max(int(rows), 1))()
    rc = lib().tkvo_calibrate_per_channel_minmax(_p(x), x.size, int(rows), int(cols),
                                                  int(symmetric), C.cast(out, C.c_void_p))
    if rc != 0:
        raise ValueError("rows/cols must be > 0 and data must hold rows*cols")
    return [QuantParams._from(out[i]) for i in range(int(rows))]


def quantize_int8_symmetric(src, scale: float, recipe: int = PRIMARY) -> np.ndarray:
    x = _f32(src)
    dst = np.zeros(x.size, dtype=np.int32)
    lib().tkvo_quantize_int8_symmetric(_p(x), x.size, _p(dst), float(np.float32(scale)), int(recipe))
    return dst


def dequantize_int8_symmetric(src, scale: float) -> np.ndarray:
    q = _i32(src)
    dst = np.zeros(q.size, dtype=np.float32)
    lib().tkvo_dequantize_int8_symmetric(_p(q), q.size, _p(dst), float(np.float32(scale)))
    return dst


def quantize_int8_per_channel(src, rows: int, cols: int, scales) -> np.ndarray:
    x = _f32(src)
    s = _f32(scales)
    dst = np.zeros(int(rows) * int(cols), dtype=np.int32)
    lib().tkvo_quantize_int8_per_channel(_p(x), _p(dst), int(rows), int(cols), _p(s))
    return dst


def dequantize_int8_per_channel(src, rows: int, cols: int, scales) -> np.ndarray:
    q = _i32(src)
    s = _f32(scales)
    dst = np.zeros(int(rows) * int(cols), dtype=np.float32)
    lib().tkvo_dequantize_int8_per_channel(_p(q), _p(dst), int(rows), int(cols), _p(s))
    return dst


def quantize_dynamic_int8_rowwise(src, rows: int, cols: int):
    x = _f32(src)
    dst = np.zeros(int(rows) * int(cols), dtype=np.int32)
    sc = np.zeros(int(rows), dtype=np.float32)
    lib().tkvo_quantize_dynamic_int8_rowwise(_p(x), _p(dst), int(rows), int(cols), _p(sc))
    return dst, sc


# ---- matmul.tkv ------------------------------------------------------------

def _bias(bias):
    if bias is None:
        return np.zeros(1, dtype=np.float32), 0
    b = _f32(bias)
    return (b if b.size else np.zeros(1, dtype=np.float32)), b.size


def matmul_int8_accum(a, w, m: int, n: int, k: int) -> np.ndarray:
    A, W = _i32(a), _i32(w)
    acc = np.zeros(int(m) * int(n), dtype=np.int32)
    lib().tkvo_matmul_int8_accum(_p(A), _p(W), _p(acc), int(m), int(n), int(k))
    return acc


def matmul_int8_symmetric(a, w, bias, m, n, k, scale_a, scale_w, recipe=PRIMARY) -> np.ndarray:
    A, W = _i32(a), _i32(w)
    b, nb = _bias(bias)
    y = np.zeros(int(m) * int(n), dtype=np.float32)
    lib().tkvo_matmul_int8_symmetric(_p(A), _p(W), _p(b), nb, _p(y), int(m), int(n), int(k),
                                     float(np.float32(scale_a)), float(np.float32(scale_w)),
                                     int(recipe))
    return y


def matmul_int8_per_channel(a, w, bias, m, n, k, scale_a, scales_w, recipe=PRIMARY,
                            threads: int = 1) -> np.ndarray:
    A, W = _i32(a), _i32(w)
    b, nb = _bias(bias)
    s = _f32(scales_w)
    if s.size < int(n):
        raise ValueError("scales_w smaller than N")
    y = np.zeros(int(m) * int(n), dtype=np.float32)
    if threads == 1:
        lib().tkvo_matmul_int8_per_channel(_p(A), _p(W), _p(b), nb, _p(y), int(m), int(n), int(k),
                                           float(np.float32(scale_a)), _p(s), s.size, int(recipe))
    else:
        lib().tkvo_matmul_int8_per_channel_mt(_p(A), _p(W), _p(b), nb, _p(y), int(m), int(n),
                                              int(k), float(np.float32(scale_a)), _p(s), s.size,
                                              int(threads))
    return y


def quantize_fp8_e4m3(src) -> np.ndarray:
    x = _f32(src)
    dst = np.zeros(x.size, dtype=np.int32)
    lib().tkvo_quantize_fp8_e4m3(_p(x), x.size, _p(dst))
    return dst


def dequantize_fp8_e4m3(src) -> np.ndarray:
    q = _i32(src)
    dst = np.zeros(q.size, dtype=np.float32)
    lib().tkvo_dequantize_fp8_e4m3(_p(q), q.size, _p(dst))
    return dst


def matmul_fp8_e4m3(a, w, bias, m, n, k) -> np.ndarray:
    A, W = _i32(a), _i32(w)
    b, nb = _bias(bias)
    y = np.zeros(int(m) * int(n), dtype=np.float32)
    lib().tkvo_matmul_fp8_e4m3(_p(A), _p(W), _p(b), nb, _p(y), int(m), int(n), int(k))
    return y


def matmul_fp8_e4m3_exact(a, w, m, n, k):
    """Exact dot sums (units of 2^-20, int64) and sum |a_k w_k| per output."""
    A, W = _i32(a), _i32(w)
    acc = np.zeros(int(m) * int(n), dtype=np.int64)
    asum = np.zeros(int(m) * int(n), dtype=np.float64)
    lib().tkvo_matmul_fp8_e4m3_exact(_p(A), _p(W), _p(acc), _p(asum), int(m), int(n), int(k))
    return acc, asum


# ---- FP8 W8A8 linear (R-ext: the scaled extension of matmul_fp8_e4m3) -------

def quantize_fp8_e4m3_dynamic_tensor(src):
    """Per-tensor FP8 activation pack: (codes, scale) with scale =
    fl32(max(am, 1e-8) / 240) and codes = encode(fl32(x * fl32(1 / scale))) - 128."""
    x = _f32(src)
    dst = np.zeros(x.size, dtype=np.int32)
    s = C.c_float()
    lib().tkvo_quantize_fp8_e4m3_dynamic_tensor(_p(x), x.size, _p(dst), C.byref(s))
    return dst, np.float32(s.value)


def fp8_weight_pack(w, rows: int, cols: int):
    """Per-output-channel FP8 weight pack: (codes [rows * cols], scales [rows])."""
    x = _f32(w)
    dst = np.zeros(int(rows) * int(cols), dtype=np.int32)
    sc = np.zeros(int(rows), dtype=np.float32)
    lib().tkvo_fp8_weight_pack(_p(x), int(rows), int(cols), _p(dst), _p(sc))
    return dst, sc


def matmul_fp8_e4m3_scaled(a, w, bias, m, n, k, scale_a, scales_w, per_token=False):
    """y = fl32(fl64(fl64(S * sa) * sw[n]) + b[n]), S the exact product sum;
    scale_a is one value (per tensor) or m values (per_token=True)."""
    A, W = _i32(a), _i32(w)
    b, nb = _bias(bias)
    sa = _f32(np.atleast_1d(scale_a))
    sw = _f32(scales_w)
    y = np.zeros(int(m) * int(n), dtype=np.float32)
    lib().tkvo_matmul_fp8_e4m3_scaled(_p(A), _p(W), _p(b), nb, _p(y), int(m), int(n), int(k),
                                      _p(sa), 1 if per_token else 0, _p(sw))
    return y


# ---- session.tkv nodes -----------------------------------------------------

def matmul_integer(a, b, y_len, m, n, k) -> np.ndarray:
    A, B = _i32(a), _i32(b)
    y = np.zeros(max(int(y_len), 1), dtype=np.int64)
    lib().tkvo_matmul_integer(_p(A), A.size, _p(B), B.size, _p(y), int(y_len),
                              int(m), int(n), int(k))
    return y[: int(y_len)]


def qlinear_matmul(a, sa, zpa, b, sw, zpw, sy, zpy, y_len, m, n, k,
                   recipe: int = PRIMARY) -> np.ndarray:
    A, B = _i32(a), _i32(b)
    y = np.zeros(max(int(y_len), 1), dtype=np.int32)
    lib().tkvo_qlinear_matmul(_p(A), A.size, float(np.float32(sa)), int(zpa), _p(B), B.size,
                              float(np.float32(sw)), int(zpw), float(np.float32(sy)), int(zpy),
                              _p(y), int(y_len), int(m), int(n), int(k), int(recipe))
    return y[: int(y_len)]


def quantize_linear(x, scales, zero_point=0, outer=1, dim=1, inner=1) -> np.ndarray:
    X, S = _f32(x), _f32(scales)
    y = np.zeros(X.size, dtype=np.int32)
    lib().tkvo_quantize_linear(_p(X), X.size, _p(S), S.size, int(zero_point), int(outer),
                               int(dim), int(inner), _p(y))
    return y


def dequantize_linear(x, scales, zero_point=0, outer=1, dim=1, inner=1) -> np.ndarray:
    X, S = _i32(x), _f32(scales)
    y = np.zeros(X.size, dtype=np.float32)
    lib().tkvo_dequantize_linear(_p(X), X.size, _p(S), S.size, int(zero_point), int(outer),
                                 int(dim), int(inner), _p(y))
    return y


def dynamic_quantize_linear(x):
    X = _f32(x)
    y = np.zeros(X.size, dtype=np.int32)
    ys = np.zeros(1, dtype=np.float32)
    yz = np.zeros(1, dtype=np.float32)
    rc = lib().tkvo_dynamic_quantize_linear(_p(X), X.size, _p(y), _p(ys), _p(yz))
    if rc != 0:
        raise ValueError("DynamicQuantizeLinear needs a non-empty input")
    return y, ys[0], yz[0]


def quantized_gemm_node(aq, wq, bias, m, n, k, scale_a, scale_b, scales_w, recipe=PRIMARY):
    A, W = _i32(aq), _i32(wq)
    b, nb = _bias(bias)
    s = _f32(scales_w if scales_w is not None else [])
    sp = s if s.size else np.zeros(1, dtype=np.float32)
    y = np.zeros(int(m) * int(n), dtype=np.float32)
    rc = lib().tkvo_quantized_gemm_node(_p(A), _p(W), _p(b), nb, _p(y), int(m), int(n), int(k),
                                        float(np.float32(scale_a)), float(np.float32(scale_b)),
                                        _p(sp), s.size, int(recipe))
    if rc != 0:
        raise ValueError("scales_w smaller than N")
    return y


# ---- int4.tkv: grouped INT4 -------------------------------------------------

def _i64(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.int64)


def _groups(rows: int, cols: int, group_size: int) -> int:
    return max(int(rows) * (int(cols) // int(group_size)), 1) if int(group_size) > 0 else 1


def quantize_int4_grouped(src, rows: int, cols: int, group_size: int, npacked=None):
    """(packed int32 bytes [rows * cols / 2], scales f32 [rows * cols / group_size])."""
    x = _f32(src)
    packed = np.zeros(int(npacked) if npacked is not None else max(int(rows) * (int(cols) // 2), 1),
                      np.int32)
    scales = np.zeros(_groups(rows, cols, group_size), np.float32)
    rc = lib().tkvo_quantize_int4_grouped(_p(x), x.size, int(rows), int(cols), int(group_size),
                                          _p(packed), packed.size, _p(scales))
    if rc != 0:
        raise ValueError("cols must be a multiple of group_size and even; src / packed sizes")
    return packed, scales


def dequantize_int4_grouped(packed, rows: int, cols: int, group_size: int, scales) -> np.ndarray:
    pk, sc = _i32(packed), _f32(scales)
    y = np.zeros(max(int(rows) * int(cols), 1), np.float32)
    rc = lib().tkvo_dequantize_int4_grouped(_p(pk), pk.size, _p(y), y.size, int(rows), int(cols),
                                            int(group_size), _p(sc), sc.size)
    if rc != 0:
        raise ValueError("scales smaller than rows*num_groups / dst too small")
    return y[: int(rows) * int(cols)]


def quantize_int4_grouped_asym(src, rows: int, cols: int, group_size: int):
    """(packed, scales f32, zero points int64), one scale / zero point per group."""
    x = _f32(src)
    packed = np.zeros(max(int(rows) * (int(cols) // 2), 1), np.int32)
    scales = np.zeros(_groups(rows, cols, group_size), np.float32)
    zps = np.zeros(scales.size, np.int64)
    rc = lib().tkvo_quantize_int4_grouped_asym(_p(x), x.size, int(rows), int(cols),
                                               int(group_size), _p(packed), packed.size,
                                               _p(scales), _p(zps))
    if rc != 0:
        raise ValueError("cols must be a multiple of group_size and even; src / packed sizes")
    return packed, scales, zps


def dequantize_int4_grouped_asym(packed, rows, cols, group_size, scales, zps) -> np.ndarray:
    pk, sc, zp = _i32(packed), _f32(scales), _i64(zps)
    y = np.zeros(max(int(rows) * int(cols), 1), np.float32)
    rc = lib().tkvo_dequantize_int4_grouped_asym(_p(pk), pk.size, _p(y), y.size, int(rows),
                                                 int(cols), int(group_size), _p(sc), _p(zp),
                                                 min(sc.size, zp.size))
    if rc != 0:
        raise ValueError("scales / zps smaller than rows*num_groups")
    return y[: int(rows) * int(cols)]


def permute_cols(src, rows: int, cols: int, perm, inverse: bool = False) -> np.ndarray:
    x, pm = _f32(src), _i64(perm)
    y = np.zeros(max(int(rows) * int(cols), 1), np.float32)
    rc = lib().tkvo_permute_cols(_p(x), int(rows), int(cols), _p(pm), pm.size, int(bool(inverse)),
                                 _p(y))
    if rc != 0:
        raise ValueError("perm length must equal cols")
    return y[: int(rows) * int(cols)]


def matmul_int4_grouped(a, packed_w, bias, m, n, k, group_size, scales_w, perm=None) -> np.ndarray:
    A, W, S = _f32(a), _i32(packed_w), _f32(scales_w)
    b, nb = _bias(bias)
    y = np.zeros(max(int(m) * int(n), 1), np.float32)
    pm = _i64(perm) if perm is not None else None
    rc = lib().tkvo_matmul_int4_grouped(_p(A), _p(W), _p(b), nb, _p(y),
                                        int(m), int(n), int(k), int(group_size), _p(S), S.size,
                                        _p(pm) if pm is not None else None)
    if rc != 0:
        raise ValueError("scales_w smaller than N*num_groups")
    return y[: int(m) * int(n)]


# ---- gguf.tkv: block formats -------------------------------------------------

GGUF_Q4_0, GGUF_Q4_1, GGUF_Q8_0 = 2, 3, 8


def f16_to_f32(h: int) -> np.float32:
    return np.float32(lib().tkvo_f16_to_f32(int(h)))


def dequantize_gguf(raw, n: int, dtype: int) -> np.ndarray:
    r = np.ascontiguousarray(np.frombuffer(bytes(raw), np.uint8) if not isinstance(raw, np.ndarray)
                             else raw, dtype=np.uint8)
    y = np.zeros(max(int(n), 1), np.float32)
    rc = lib().tkvo_dequantize_gguf(_p(r), r.size, int(n), int(dtype), _p(y))
    if rc != 0:
        raise ValueError("unsupported dtype or raw too short")
    return y[: int(n)]


def matmul_q8_0(a, raw, sa, m: int, n: int, k: int, bias=None) -> np.ndarray:
    """Q8_0 weights (raw blocks, n rows of k / 32) on int8 activation codes
    a [m, k] with scale sa (one value: per tensor; m values: per token).
    Extension with no reference counterpart: acc = fmaf chain over the groups
    of (float)dot_g * d, y = fl32(fl64(acc) * sa + b)."""
    A = np.ascontiguousarray(a, dtype=np.int32).reshape(-1)
    r = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    s = np.ascontiguousarray(np.atleast_1d(sa), dtype=np.float32)
    if s.size not in (1, m):
        raise ValueError("sa: one value or one per row")
    stride = 0 if s.size == 1 else 1
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.zeros((max(int(m), 1), max(int(n), 1)), np.float32)
    rc = lib().tkvo_matmul_q8_0(_p(A), _p(r), r.size, _p(s), stride, None if b is None else _p(b),
                                0 if b is None else b.size, _p(y), int(m), int(n), int(k))
    if rc != 0:
        raise ValueError("k % 32 != 0 or raw too short")
    return y[: int(m), : int(n)]
