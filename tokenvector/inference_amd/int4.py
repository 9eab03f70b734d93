"""Host-side mirror of tv/quantization/int4.tkv (grouped INT4, GPTQ / AWQ
class), running on libtkv_hip.

Same names, argument order and ValueError cases as the .tkv functions:
packed codes are int32 arrays holding one byte per entry (low nibble = even
column), ``scales_out`` / ``zps_out`` are Python lists that receive one entry
per (row, group) as the reference appends them, and the GEMMs write ``py`` in
place.  Every call goes through the C ABI to the GPU; the HIP path returns
TKV_HIP_UNSUPPORTED (raised here) only for shapes the reference's own
quantizer never produces (odd K, K not a multiple of the group size).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .quantization import _bias, _f32_in, _i32_in, _out, _p


def _i64_in(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int64).reshape(-1))


def _groups(rows: int, cols: int, group_size: int) -> int:
    return int(rows) * (int(cols) // int(group_size)) if int(group_size) > 0 else 0


def quantize_int4_grouped(src, rows: int, cols: int, group_size: int, packed_out: np.ndarray,
                          scales_out: list) -> int:
    """int4.tkv:36-57: symmetric grouped INT4, scales appended to scales_out."""
    x, pk = _f32_in(src), _out(packed_out, np.int32)
    ng = _groups(rows, cols, group_size)
    sc = np.zeros(max(ng, 1), np.float32)
    _lib.check(_lib.lib().tkv_hip_quantize_int4_grouped(
        _p(x), x.size, int(rows), int(cols), int(group_size), _p(pk), pk.size, _p(sc), ng))
    scales_out.extend(np.float32(v) for v in sc[:ng])
    return 0


def dequantize_int4_grouped(packed, dst: np.ndarray, rows: int, cols: int, group_size: int,
                            scales) -> int:
    """int4.tkv:60-73."""
    pk, y, sc = _i32_in(packed), _out(dst, np.float32), _f32_in(scales)
    _lib.check(_lib.lib().tkv_hip_dequantize_int4_grouped(
        _p(pk), pk.size, _p(y), y.size, int(rows), int(cols), int(group_size), _p(sc), sc.size))
    return 0


def quantize_int4_grouped_asym(src, rows: int, cols: int, group_size: int,
                               packed_out: np.ndarray, scales_out: list, zps_out: list) -> int:
    """int4.tkv:77-157: AWQ-style asymmetric grouped INT4."""
    x, pk = _f32_in(src), _out(packed_out, np.int32)
    ng = _groups(rows, cols, group_size)
    sc = np.zeros(max(ng, 1), np.float32)
    zp = np.zeros(max(ng, 1), np.int64)
    _lib.check(_lib.lib().tkv_hip_quantize_int4_grouped_asym(
        _p(x), x.size, int(rows), int(cols), int(group_size), _p(pk), pk.size, _p(sc), _p(zp), ng))
    scales_out.extend(np.float32(v) for v in sc[:ng])
    zps_out.extend(int(v) for v in zp[:ng])
    return 0


def dequantize_int4_grouped_asym(packed, dst: np.ndarray, rows: int, cols: int,
                                 group_size: int, scales, zps) -> int:
    """int4.tkv:160-170."""
    pk, y, sc, zp = _i32_in(packed), _out(dst, np.float32), _f32_in(scales), _i64_in(zps)
    _lib.check(_lib.lib().tkv_hip_dequantize_int4_grouped_asym(
        _p(pk), pk.size, _p(y), y.size, int(rows), int(cols), int(group_size), _p(sc), _p(zp),
        min(sc.size, zp.size)))
    return 0


def _permute(fn, src, rows: int, cols: int, perm) -> np.ndarray:
    x, pm = _f32_in(src), _i64_in(perm)
    out = np.zeros(max(int(rows) * int(cols), 1), np.float32)
    _lib.check(fn(_p(x), x.size, int(rows), int(cols), _p(pm), pm.size, _p(out), out.size))
    return out[: int(rows) * int(cols)]


def permute_cols(src, rows: int, cols: int, perm) -> np.ndarray:
    """int4.tkv:175-182: out[r, c] = src[r, perm[c]]."""
    return _permute(_lib.lib().tkv_hip_permute_cols, src, rows, cols, perm)


def inv_permute_cols(src, rows: int, cols: int, perm) -> np.ndarray:
    """int4.tkv:185-192: out[r, perm[c]] = src[r, c]."""
    return _permute(_lib.lib().tkv_hip_inv_permute_cols, src, rows, cols, perm)


def matmul_int4_grouped(pa, packed_w, pbias, py: np.ndarray, m, n, k, group_size,
                        scales_w) -> int:
    """int4.tkv:218-239: Y = A_f32 . W_int4^T + bias, per-group scales."""
    a, w, sw, y = _f32_in(pa), _i32_in(packed_w), _f32_in(scales_w), _out(py, np.float32)
    b, nb = _bias(pbias)
    _lib.check(_lib.lib().tkv_hip_matmul_int4_grouped(
        _p(a), a.size, _p(w), w.size, _p(b), nb, _p(y), y.size, int(m), int(n), int(k),
        int(group_size), _p(sw), sw.size))
    return 0


def matmul_int4_grouped_ordered(pa, packed_w, pbias, py: np.ndarray, m, n, k, group_size,
                                scales_w, perm) -> int:
    """int4.tkv:195-215: the act-order form (activation column perm[k])."""
    a, w, sw, y = _f32_in(pa), _i32_in(packed_w), _f32_in(scales_w), _out(py, np.float32)
    pm = _i64_in(perm)
    b, nb = _bias(pbias)
    _lib.check(_lib.lib().tkv_hip_matmul_int4_grouped_ordered(
        _p(a), a.size, _p(w), w.size, _p(b), nb, _p(y), y.size, int(m), int(n), int(k),
        int(group_size), _p(sw), sw.size, _p(pm), pm.size))
    return 0
