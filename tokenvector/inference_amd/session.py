"""Mirror of the reference graph runtime's quantized nodes on libtkv_hip.

``QuantNode`` carries the ``ExecutionNode`` fields these ops read
(tv/runtime/session.tkv:460-558: scale_a, scale_b, scales_w, qlinear_axis)
and dispatches exactly as ``ExecutionNode.execute`` does for:

    OperatorType_QuantizedGemm (21)          session.tkv:678-697
    OperatorType_QuantizeLinear (63)         session.tkv:1896-1953
    OperatorType_DequantizeLinear (64)       session.tkv:1955-1990
    OperatorType_QLinearMatMul (65)          session.tkv:1992-2071
    OperatorType_MatMulInteger (78)          session.tkv:2789-2851
    OperatorType_DynamicQuantizeLinear (79)  session.tkv:2853-2901

Inputs are (array, shape) pairs in the node's input order; dims follow
``_m`` / ``_k_gemm`` / ``_n_gemm`` (session.tkv:3029-3051).  The graph,
arena and session around the nodes stay the reference's.
"""
from __future__ import annotations

import ctypes as C
from typing import List, Sequence, Tuple

import numpy as np

from . import _lib

OperatorType_QuantizedGemm = 21
OperatorType_QuantizeLinear = 63
OperatorType_DequantizeLinear = 64
OperatorType_QLinearMatMul = 65
OperatorType_MatMulInteger = 78
OperatorType_DynamicQuantizeLinear = 79

Tensor = Tuple[np.ndarray, Sequence[int]]


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))


def _i32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32).reshape(-1))


def _count(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


class QuantNode:
    """The quantized-op subset of ExecutionNode (session.tkv:460-558)."""

    def __init__(self, name: str, op: int):
        self.name = name
        self.op_type = int(op)
        self.scale_a = np.float32(1.0)
        self.scale_b = np.float32(1.0)
        self.scales_w: List[float] = []
        self.qlinear_axis = 1

    # session.tkv:3029-3051
    @staticmethod
    def _m(a_shape) -> int:
        return int(a_shape[0]) if len(a_shape) > 1 else 1

    @staticmethod
    def _k_gemm(a_shape) -> int:
        return int(a_shape[1]) if len(a_shape) > 1 else _count(a_shape)

    @staticmethod
    def _n_gemm(b_shape) -> int:
        return int(b_shape[0]) if len(b_shape) > 1 else _count(b_shape)

    def execute(self, inputs: List[Tensor], out_shapes: List[Sequence[int]]) -> List[np.ndarray]:
        op = self.op_type
        if op == OperatorType_QuantizedGemm:
            return [self._quantized_gemm(inputs, out_shapes[0])]
        if op == OperatorType_QuantizeLinear:
            return [self._quantize_linear(inputs)]
        if op == OperatorType_DequantizeLinear:
            return [self._dequantize_linear(inputs)]
        if op == OperatorType_MatMulInteger:
            return [self._matmul_integer(inputs, out_shapes[0])]
        if op == OperatorType_QLinearMatMul:
            return [self._qlinear_matmul(inputs, out_shapes[0])]
        if op == OperatorType_DynamicQuantizeLinear:
            return list(self._dynamic_quantize_linear(inputs))
        raise NotImplementedError(f"op {op} is not a quantized node")

    def _quantized_gemm(self, inputs, y_shape) -> np.ndarray:
        (aq, a_shape), (wq, w_shape) = inputs[0], inputs[1]
        m, k, n = self._m(a_shape), self._k_gemm(a_shape), self._n_gemm(w_shape)
        a, w = _i32(aq), _i32(wq)
        bias = _f32(inputs[2][0]) if len(inputs) > 2 else np.zeros(0, np.float32)
        y = np.zeros(max(_count(y_shape), m * n), np.float32)
        if a.size < m * k or w.size < n * k:
            raise IndexError("QuantizedGemm operand shorter than its shape")
        sw = _f32(self.scales_w)
        bp = bias if bias.size else np.zeros(1, np.float32)
        swp = sw if sw.size else np.zeros(1, np.float32)
        if sw.size > 0 and sw.size < n:
            raise ValueError("scales_w smaller than N")
        _lib.check(_lib.lib().tkv_hip_quantized_gemm(
            _p(a), _p(w), _p(bp), bias.size, _p(y), m, n, k, float(np.float32(self.scale_a)),
            float(np.float32(self.scale_b)), _p(swp), sw.size))
        return y[: _count(y_shape)] if _count(y_shape) else y

    def _axis_view(self, shape):
        rank = len(shape)
        ax = self.qlinear_axis if self.qlinear_axis >= 0 else self.qlinear_axis + rank
        outer = _count(shape[:ax])
        dim = int(shape[ax])
        inner = _count(shape[ax + 1:])
        return outer, dim, inner

    @staticmethod
    def _zero_point(inputs) -> int:
        # zp = int(_span0(arena, ...)): first element of a float span, truncated
        return int(np.float32(_f32(inputs[2][0])[0])) if len(inputs) > 2 else 0

    def _quantize_linear(self, inputs) -> np.ndarray:
        (x, x_shape), (sc, _) = inputs[0], inputs[1]
        x, s = _f32(x), _f32(sc)
        zp = self._zero_point(inputs)
        outer, dim, inner = (1, 1, 1) if s.size == 1 else self._axis_view(x_shape)
        y = np.zeros(x.size, np.int32)
        _lib.check(_lib.lib().tkv_hip_quantize_linear(_p(x), x.size, _p(s), s.size, zp, outer,
                                                      dim, inner, _p(y)))
        return y

    def _dequantize_linear(self, inputs) -> np.ndarray:
        (x, x_shape), (sc, _) = inputs[0], inputs[1]
        x, s = _i32(x), _f32(sc)
        zp = self._zero_point(inputs)
        outer, dim, inner = (1, 1, 1) if s.size == 1 else self._axis_view(x_shape)
        y = np.zeros(x.size, np.float32)
        _lib.check(_lib.lib().tkv_hip_dequantize_linear(_p(x), x.size, _p(s), s.size, zp, outer,
                                                        dim, inner, _p(y)))
        return y

    def _matmul_integer(self, inputs, y_shape) -> np.ndarray:
        (a, a_shape), (b, b_shape) = inputs[0], inputs[1]
        a, b = _i32(a), _i32(b)
        # session.tkv:2809-2819 (note: a 1-D A gives m = K)
        m = int(a_shape[0]) if len(a_shape) > 0 else 1
        k = int(a_shape[1]) if len(a_shape) > 1 else _count(a_shape)
        n = int(b_shape[1]) if len(b_shape) > 1 else _count(b_shape)
        ny = _count(y_shape)
        y = np.zeros(max(ny, 1), np.int64)
        _lib.check(_lib.lib().tkv_hip_matmul_integer(_p(a), a.size, _p(b), b.size, _p(y), ny,
                                                     m, n, k))
        return y[:ny]

    def _qlinear_matmul(self, inputs, y_shape, recipe: int = 0) -> np.ndarray:
        """Inputs a, a_scale, a_zero_point, b, b_scale, b_zero_point, y_scale,
        y_zero_point (session.tkv:1994-2014): scalars are the first element of
        a float tensor, zero points truncated to integers by int()."""
        (a, a_shape), (b, b_shape) = inputs[0], inputs[3]
        a, b = _i32(a), _i32(b)

        def scalar(t):
            return np.float32(np.asarray(t[0], dtype=np.float32).reshape(-1)[0])

        sa, sw, sy = scalar(inputs[1]), scalar(inputs[4]), scalar(inputs[6])
        zpa, zpw, zpy = int(scalar(inputs[2])), int(scalar(inputs[5])), int(scalar(inputs[7]))
        m = int(a_shape[0]) if len(a_shape) > 1 else 1
        k = int(a_shape[1]) if len(a_shape) > 1 else _count(a_shape)
        n = int(b_shape[1]) if len(b_shape) > 1 else _count(b_shape)
        ny = _count(y_shape)
        y = np.zeros(max(ny, 1), np.int32)
        _lib.check(_lib.lib().tkv_hip_qlinear_matmul(
            _p(a), a.size, float(sa), zpa, _p(b), b.size, float(sw), zpw, float(sy), zpy, _p(y),
            ny, m, n, k, int(recipe)))
        return y[:ny]

    def _dynamic_quantize_linear(self, inputs):
        x = _f32(inputs[0][0])
        y = np.zeros(x.size, np.int32)
        ys, yz = C.c_float(), C.c_float()
        _lib.check(_lib.lib().tkv_hip_dynamic_quantize_linear(_p(x), x.size, _p(y), C.byref(ys),
                                                              C.byref(yz)))
        return y, np.array([ys.value], np.float32), np.array([yz.value], np.float32)


def new_node(name: str, op: int) -> QuantNode:
    """session.tkv new_node for the quantized op types."""
    return QuantNode(name, op)
