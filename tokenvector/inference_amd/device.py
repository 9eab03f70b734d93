"""Device-pointer side of libtkv_hip: contexts, buffers, the packed-code
kernels and the resident quantized weight / linear.

These wrap the ``tkv_hip_dev_*`` / ``tkv_hip_weight_*`` entry points, which
take device pointers and run asynchronously on the context's stream.  Device
memory comes from the library itself (``tkv_hip_malloc``), so no framework is
needed to drive the GPU path.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np

from . import _lib

ACT_PER_TENSOR = 0
ACT_PER_TOKEN = 1
WEIGHT_INT8 = 0
WEIGHT_FP8 = 1
WEIGHT_FP8_FAST = 2
WEIGHT_Q8_0 = 3      # GGUF Q8_0 blocks on the INT8 GEMM with group scales (extension)


def _vp(x) -> C.c_void_p:
    if x is None:
        return C.c_void_p(0)
    if isinstance(x, DeviceBuffer):
        return C.c_void_p(x.ptr)
    return C.c_void_p(int(x))


# Tuning knobs of Context.set_tuning (tkv_hip.h, TKV_HIP_TUNE_*).
TUNE_GEMM_CFG = 0
TUNE_GEMM_STAGGER = 1
TUNE_DECODE_GROUP = 2
TUNE_QUANT_TWO_PASS = 3
TUNE_INT4_GEMV_WAVE = 4
TUNE_GRID_SPIN = 5
TUNE_DECODE_DMA = 6


class Context:
    """A libtkv_hip context: one HIP stream plus grow-only workspaces."""

    def __init__(self, device: int = 0):
        h = C.c_int64()
        _lib.check(_lib.lib().tkv_hip_ctx_create(int(device), C.byref(h)))
        self.handle = h.value

    def synchronize(self) -> None:
        _lib.check(_lib.lib().tkv_hip_ctx_synchronize(self.handle))

    def set_tuning(self, knob: int, value: int) -> None:
        """Tuning / test override of this context (TKV_HIP_TUNE_*; -1 = automatic)."""
        _lib.check(_lib.lib().tkv_hip_ctx_set_tuning(self.handle, int(knob), int(value)))

    def retired_buffers(self) -> int:
        """Workspace buffers kept alive for this context's live graphs."""
        n = C.c_int64()
        _lib.check(_lib.lib().tkv_hip_ctx_retired_buffers(self.handle, C.byref(n)))
        return n.value

    def close(self) -> None:
        if self.handle:
            _lib.check(_lib.lib().tkv_hip_ctx_destroy(self.handle))
            self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class DeviceBuffer:
    """A device allocation owned by Python (freed on close / GC)."""

    def __init__(self, ctx: Context, nbytes: int, dtype=np.uint8, shape=None):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape) if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = C.c_void_p()
        _lib.check(_lib.lib().tkv_hip_malloc(ctx.handle, self.nbytes, C.byref(p)))
        self.ptr = p.value or 0

    @classmethod
    def empty(cls, ctx: Context, shape, dtype) -> "DeviceBuffer":
        shape = (shape,) if np.isscalar(shape) else tuple(shape)
        n = int(np.prod(shape)) if len(shape) else 1
        return cls(ctx, n * np.dtype(dtype).itemsize, dtype, shape)

    @classmethod
    def from_host(cls, ctx: Context, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = cls(ctx, arr.nbytes, arr.dtype, arr.shape)
        b.upload(arr)
        return b

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError("host array larger than device buffer")
        _lib.check(_lib.lib().tkv_hip_memcpy_h2d(self.ctx.handle, C.c_void_p(self.ptr),
                                                 arr.ctypes.data_as(C.c_void_p), arr.nbytes))

    def copy_from(self, src: "DeviceBuffer", nbytes: Optional[int] = None) -> None:
        """Device-to-device copy on the context's stream (asynchronous)."""
        n = self.nbytes if nbytes is None else int(nbytes)
        if n > self.nbytes or n > src.nbytes:
            raise ValueError("copy larger than a buffer")
        _lib.check(_lib.lib().tkv_hip_memcpy_d2d(self.ctx.handle, C.c_void_p(self.ptr),
                                                 C.c_void_p(src.ptr), n))

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        _lib.check(_lib.lib().tkv_hip_memcpy_d2h(self.ctx.handle, out.ctypes.data_as(C.c_void_p),
                                                 C.c_void_p(self.ptr), out.nbytes))
        return out

    def close(self) -> None:
        if self.ptr:
            _lib.check(_lib.lib().tkv_hip_free(self.ctx.handle, C.c_void_p(self.ptr)))
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def params_buffer(ctx: Context) -> DeviceBuffer:
    """Room for one tkv_hip_qparams_dev."""
    return DeviceBuffer(ctx, C.sizeof(_lib.QParamsDev), np.uint8)


def read_params(buf: DeviceBuffer) -> _lib.QParamsDev:
    raw = buf.download()
    return _lib.QParamsDev.from_buffer_copy(raw.tobytes()[: C.sizeof(_lib.QParamsDev)])


class Event:
    """HIP event on a context's stream (timing)."""

    def __init__(self):
        h = C.c_int64()
        _lib.check(_lib.lib().tkv_hip_event_create(C.byref(h)))
        self.handle = h.value

    def record(self, ctx: Context) -> None:
        _lib.check(_lib.lib().tkv_hip_event_record(ctx.handle, self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _lib.check(_lib.lib().tkv_hip_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            _lib.lib().tkv_hip_event_destroy(self.handle)
        except Exception:
            pass


class Graph:
    """The device entry points called inside ``with Graph(ctx) as g:``,
    captured from the context's stream into one replayable HIP graph.

    Every call inside the block must have run once, with the same sizes,
    before the capture (workspaces are sized then); ``g.launch()`` replays
    the sequence on the context's stream with the captured pointers."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.handle = 0

    def __enter__(self):
        _lib.check(_lib.lib().tkv_hip_capture_begin(self.ctx.handle))
        return self

    def __exit__(self, exc_type, exc, tb):
        h = C.c_int64()
        rc = _lib.lib().tkv_hip_capture_end(self.ctx.handle, C.byref(h))
        if exc_type is None:
            _lib.check(rc)
        self.handle = h.value
        return False

    def launch(self) -> None:
        _lib.check(_lib.lib().tkv_hip_graph_launch(self.ctx.handle, self.handle))

    def close(self) -> None:
        if self.handle:
            _lib.check(_lib.lib().tkv_hip_graph_destroy(self.handle))
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def memset(ctx: Context, dst, value: int, nbytes: int) -> None:
    """Byte fill on the context's stream (a kernel: capturable)."""
    _lib.check(_lib.lib().tkv_hip_memset(ctx.handle, _vp(dst), int(value), int(nbytes)))


# ---- packed-code kernels (device pointers) ---------------------------------

def calibrate_minmax(ctx, x, n, symmetric, params) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_calibrate_minmax(ctx.handle, _vp(x), int(n), int(symmetric),
                                                       _vp(params)))


def calibrate_kl(ctx, x, n, params, num_bins: int = 2048, target_bins: int = 128) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_calibrate_kl(ctx.handle, _vp(x), int(n), int(num_bins),
                                                   int(target_bins), _vp(params)))


def calibrate_percentile(ctx, x, n, params, percentile: float = 99.99, symmetric: int = 1) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_calibrate_percentile(
        ctx.handle, _vp(x), int(n), float(np.float32(percentile)), int(symmetric), _vp(params)))


def calibrate_mse(ctx, x, n, params, num_candidates: int = 50) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_calibrate_mse(ctx.handle, _vp(x), int(n),
                                                    int(num_candidates), _vp(params)))


def calibrate_rows(ctx, x, rows, cols, scales) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_calibrate_rows(ctx.handle, _vp(x), int(rows), int(cols),
                                                     _vp(scales)))


def quantize_int8_tensor(ctx, x, n, params, q) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_quantize_int8_tensor(ctx.handle, _vp(x), int(n),
                                                           _vp(params), _vp(q)))


def quantize_int8_dynamic_tensor(ctx, x, n, q, params) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_quantize_int8_dynamic_tensor(ctx.handle, _vp(x), int(n),
                                                                   _vp(q), _vp(params)))


def quantize_int8_per_channel(ctx, x, rows, cols, scales, q) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_quantize_int8_per_channel(ctx.handle, _vp(x), int(rows),
                                                                int(cols), _vp(scales), _vp(q)))


def quantize_dynamic_int8_rowwise(ctx, x, rows, cols, q, scales_out) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_quantize_dynamic_int8_rowwise(
        ctx.handle, _vp(x), int(rows), int(cols), _vp(q), _vp(scales_out)))


def dequantize_int8(ctx, q, rows, cols, scale, scales, y) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_dequantize_int8(ctx.handle, _vp(q), int(rows), int(cols),
                                                      float(scale), _vp(scales), _vp(y)))


def quantize_fp8_e4m3(ctx, x, n, q) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_quantize_fp8_e4m3(ctx.handle, _vp(x), int(n), _vp(q)))


def quantize_fp8_e4m3_scaled(ctx, x, n, params, q) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_quantize_fp8_e4m3_scaled(ctx.handle, _vp(x), int(n),
                                                               _vp(params), _vp(q)))


def quantize_fp8_e4m3_dynamic_tensor(ctx, x, n, q, params) -> None:
    """Per-tensor FP8 activation quantize (extension): scale = max|x| / 240."""
    _lib.check(_lib.lib().tkv_hip_dev_quantize_fp8_e4m3_dynamic_tensor(ctx.handle, _vp(x), int(n),
                                                                       _vp(q), _vp(params)))


def dequantize_fp8_e4m3(ctx, q, n, y) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_dequantize_fp8_e4m3(ctx.handle, _vp(q), int(n), _vp(y)))


def matmul_int8(ctx, a, w, m, n, k, scale_a, scale_a_stride, scale_w, scales_w, bias, y,
                recipe=0) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_matmul_int8(ctx.handle, _vp(a), _vp(w), int(m), int(n),
                                                  int(k), _vp(scale_a), int(scale_a_stride),
                                                  float(scale_w), _vp(scales_w), _vp(bias),
                                                  _vp(y), int(recipe)))


def matmul_q8_0(ctx, a, codes, group_scales, m, n, k, scale_a, scale_a_stride, bias, y) -> None:
    """Q8_0 weights on int8 activation codes (extension; no reference
    counterpart): a [m,k], codes [n,k] int8, group_scales f32 [n, k/32];
    acc = fma chain over the groups of float(dot_g) * d, y = acc * sa + bias."""
    _lib.check(_lib.lib().tkv_hip_dev_matmul_q8_0(ctx.handle, _vp(a), _vp(codes),
                                                  _vp(group_scales), int(m), int(n), int(k),
                                                  _vp(scale_a), int(scale_a_stride), _vp(bias),
                                                  _vp(y)))


def qlinear_matmul(ctx, a, sa, zpa, w, sw, zpw, sy, zpy, y, m, n, k, recipe: int = 0) -> None:
    """QLinearMatMul on int8 codes: a [m,k], w [n,k] (B transposed), y int8 [m,n]."""
    _lib.check(_lib.lib().tkv_hip_dev_qlinear_matmul(
        ctx.handle, _vp(a), float(sa), int(zpa), _vp(w), float(sw), int(zpw), float(sy),
        int(zpy), _vp(y), int(m), int(n), int(k), int(recipe)))


def matmul_int8_accum(ctx, a, w, m, n, k, acc) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_matmul_int8_accum(ctx.handle, _vp(a), _vp(w), int(m), int(n),
                                                        int(k), _vp(acc)))


def matmul_fp8_e4m3(ctx, a, w, m, n, k, scale_a, scale_a_stride, scales_w, bias, y,
                    fast: bool = False) -> None:
    """FP8 GEMM on raw e4m3 bytes; fast=True runs the full-rate FP8 MFMA
    (stated tolerance), otherwise the reference decoder's products."""
    fn = (_lib.lib().tkv_hip_dev_matmul_fp8_e4m3_fast if fast
          else _lib.lib().tkv_hip_dev_matmul_fp8_e4m3)
    _lib.check(fn(ctx.handle, _vp(a), _vp(w), int(m), int(n), int(k), _vp(scale_a),
                  int(scale_a_stride), _vp(scales_w), _vp(bias), _vp(y)))


# ---- grouped INT4 / GGUF blocks (device pointers) ---------------------------

def quantize_int4_grouped(ctx, src, rows, cols, group_size, packed, scales, zps=None) -> None:
    """packed: bytes [rows, cols / 2]; zps given selects the AWQ-asym form."""
    _lib.check(_lib.lib().tkv_hip_dev_quantize_int4_grouped(
        ctx.handle, _vp(src), int(rows), int(cols), int(group_size), _vp(packed), _vp(scales),
        _vp(zps)))


def dequantize_int4_grouped(ctx, packed, rows, cols, group_size, scales, zps, dst) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_dequantize_int4_grouped(
        ctx.handle, _vp(packed), int(rows), int(cols), int(group_size), _vp(scales), _vp(zps),
        _vp(dst)))


def permute_cols(ctx, src, rows, cols, perm, inverse, out) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_permute_cols(ctx.handle, _vp(src), int(rows), int(cols),
                                                   _vp(perm), int(bool(inverse)), _vp(out)))


def matmul_int4_grouped(ctx, a, packed_w, scales_w, bias, perm, y, m, n, k, group_size) -> None:
    """y[m, n] = a[m, k] . W_int4[n, k]^T + bias with f64 accumulation."""
    _lib.check(_lib.lib().tkv_hip_dev_matmul_int4_grouped(
        ctx.handle, _vp(a), _vp(packed_w), _vp(scales_w), _vp(bias), _vp(perm), _vp(y), int(m),
        int(n), int(k), int(group_size)))


def dequantize_gguf(ctx, raw, n, dtype, out) -> None:
    _lib.check(_lib.lib().tkv_hip_dev_dequantize_gguf(ctx.handle, _vp(raw), int(n), int(dtype),
                                                      _vp(out)))


class QuantizedLinear:
    """A device-resident quantized weight [N, K] (+ bias) and its forward."""

    def __init__(self, ctx: Context, handle: int):
        self.ctx = ctx
        self.handle = handle
        codes, scales, bias = C.c_void_p(), C.c_void_p(), C.c_void_p()
        n, k, fmt = C.c_int64(), C.c_int64(), C.c_int32()
        _lib.check(_lib.lib().tkv_hip_weight_info(handle, C.byref(codes), C.byref(scales),
                                                  C.byref(bias), C.byref(n), C.byref(k),
                                                  C.byref(fmt)))
        self.codes, self.scales, self.bias = codes.value, scales.value, bias.value
        self.n, self.k, self.format = n.value, k.value, fmt.value

    @classmethod
    def from_float(cls, ctx: Context, w, n: int, k: int, bias=None,
                   fmt: int = WEIGHT_INT8) -> "QuantizedLinear":
        h = C.c_int64()
        _lib.check(_lib.lib().tkv_hip_weight_create(ctx.handle, _vp(w), int(n), int(k), _vp(bias),
                                                    int(fmt), C.byref(h)))
        return cls(ctx, h.value)

    @classmethod
    def from_int8(cls, ctx: Context, codes, scales, n: int, k: int, bias=None) -> "QuantizedLinear":
        h = C.c_int64()
        _lib.check(_lib.lib().tkv_hip_weight_create_int8(ctx.handle, _vp(codes), _vp(scales), int(n),
                                                         int(k), _vp(bias), C.byref(h)))
        return cls(ctx, h.value)

    @classmethod
    def from_gguf_q8_0(cls, ctx: Context, raw, n: int, k: int, bias=None) -> "QuantizedLinear":
        """A weight [n, k] from raw GGUF Q8_0 blocks on the device (n rows of
        k / 32 blocks of 34 bytes); `scales` is then the group scales [n, k/32]
        with k the padded row stride."""
        h = C.c_int64()
        _lib.check(_lib.lib().tkv_hip_weight_create_gguf_q8_0(ctx.handle, _vp(raw), int(n), int(k),
                                                              _vp(bias), C.byref(h)))
        return cls(ctx, h.value)

    def forward(self, x, m: int, y, act_mode: int = ACT_PER_TENSOR) -> None:
        _lib.check(_lib.lib().tkv_hip_linear_forward(self.ctx.handle, self.handle, _vp(x), int(m),
                                                     int(act_mode), _vp(y)))

    def close(self) -> None:
        if self.handle:
            _lib.check(_lib.lib().tkv_hip_weight_free(self.handle))
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
