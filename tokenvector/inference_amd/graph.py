"""QDQ folding onto the quantized GEMM, behind the reference runtime's graph-pass API.

The reference's ``QdqFoldPass`` (tv/runtime/session.tkv:3774-3805) removes every
QuantizeLinear -> DequantizeLinear pair that are adjacent in node order and rewires their
consumers to the float input, so the MatMul / Gemm after them runs in f32 on unquantized
values.  ``QdqFoldPass`` here does that too, for every pair it cannot fold, but first turns
the QDQ pairs that feed a MatMul (1), FusedLinear (2) or Gemm (41) into the reference's own
quantized GEMM node, ``OperatorType_QuantizedGemm`` (21, session.tkv:678-697), which runs on
``tkv_hip_quantized_gemm``:

    x -> Q(sx_q) -> DQ(sx) --\\
    W -> Q(sw_q) -> DQ(sw) ---> MatMul / Gemm (+ bias C) -> y
becomes
    x -> Q(sx_q) -> QuantizedGemm(scale_a = sx, scales_w = sw | scale_b = sw, W codes [N, K], C) -> y

Foldable when: the activation DQ has a per-tensor scale, the weight DQ a per-tensor scale or
one scale per output column on B's N axis, both DQ zero points are 0 (QuantizedGemm has none;
a Q's zero point is already in its codes),
A is rank 2, the weight is an int8 initializer or a Q of a float initializer (quantized here,
once, by the Q node's own kernel), and the node is a plain product: FusedLinear without an
activation; Gemm with alpha = 1, trans_a = 0 and, with a C input, beta = 1 and C of N
elements.  B's layout follows the reference's node: MatMul / FusedLinear read [N, K] when
B's second dimension equals K and [K, N] otherwise (``_exec_linear``, session.tkv:736-773);
[K, N] codes are stored transposed.  Gemm (``_exec_gemm``, session.tkv:812-868) always takes
N from B's second dimension and, with ``trans_b``, reads b[j * B.shape[0] + p]: that is the
[N, K] product only for a square B, so a ``trans_b`` Gemm folds only when B is square
(otherwise it keeps the reference's own node, which reads B that way).

The folded node computes the QDQ graph's value with exact integer sums and the reference's
per-channel epilogue: y = fl32(fl64(fl64(Σ qx qw · sx) · sw[n]) + b[n]).  The f32 float path
computes the same sum of dequantized products with f32 rounding, so the two agree within
    |y_fold - y_float| <= 2^-24 |y_fold| + (K + 4) 2^-24 (Σ_k |dqx_k| |dqw_k| + |b|)
(one rounding per dequantized operand and per product, the f32 summation bound and the
final rounding); the reference never computes these numbers itself.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import numpy as np

from .session import (OperatorType_DequantizeLinear, OperatorType_DynamicQuantizeLinear,
                      OperatorType_MatMulInteger, OperatorType_QLinearMatMul,
                      OperatorType_QuantizedGemm, OperatorType_QuantizeLinear, QuantNode, _count)

OperatorType_MatMul = 1
OperatorType_FusedLinear = 2
OperatorType_Gemm = 41
ActivationFunction_None = 0

# ops run_graph executes; everything else belongs to the rest of the runtime
_QUANT_OPS = {OperatorType_QuantizedGemm, OperatorType_QuantizeLinear,
              OperatorType_DequantizeLinear, OperatorType_QLinearMatMul,
              OperatorType_MatMulInteger, OperatorType_DynamicQuantizeLinear}


class TensorDesc:
    """The fields of session.tkv:296-310 the passes read."""

    def __init__(self, name: str, shape: Sequence[int]):
        self.name = name
        self.shape = [int(d) for d in shape]


class ExecutionNode(QuantNode):
    """QuantNode plus the graph wiring and GEMM attributes of session.tkv:460-565."""

    def __init__(self, name: str, op: int):
        super().__init__(name, op)
        self.inputs: List[str] = []
        self.outputs: List[str] = []
        self.activation = ActivationFunction_None
        self.alpha = np.float32(1.0)
        self.beta = np.float32(1.0)
        self.trans_a = 0
        self.trans_b = 0


def new_node(name: str, op: int, inputs=(), outputs=()) -> ExecutionNode:
    n = ExecutionNode(name, op)
    n.inputs = list(inputs)
    n.outputs = list(outputs)
    return n


class ExecutionGraph:
    """The ExecutionGraph fields of session.tkv:3141-3165 the passes use:
    ``initializers`` hold f32 values, ``initializers_int8`` integer codes."""

    def __init__(self, name: str = "TokenVectorGraph"):
        self.name = name
        self.nodes: List[ExecutionNode] = []
        self.tensors: Dict[str, TensorDesc] = {}
        self.inputs: List[str] = []
        self.outputs: List[str] = []
        self.initializers: Dict[str, np.ndarray] = {}
        self.initializers_int8: Dict[str, np.ndarray] = {}

    def get_or_create_tensor(self, name: str, shape: Sequence[int] = ()) -> TensorDesc:
        if name in self.tensors:
            d = self.tensors[name]
            if len(shape) > 0 and len(d.shape) == 0:
                d.shape = [int(s) for s in shape]
            return d
        d = TensorDesc(name, shape)
        self.tensors[name] = d
        return d

    def add_initializer(self, name: str, values, shape: Sequence[int]) -> None:
        self.initializers[name] = np.ascontiguousarray(np.asarray(values, np.float32).reshape(-1))
        self.get_or_create_tensor(name, shape)

    def add_initializer_int8(self, name: str, codes, shape: Sequence[int]) -> None:
        self.initializers_int8[name] = np.ascontiguousarray(np.asarray(codes, np.int32).reshape(-1))
        self.get_or_create_tensor(name, shape)

    def add_node(self, node: ExecutionNode, out_shapes: Sequence[Sequence[int]] = ()) -> None:
        self.nodes.append(node)
        for i, o in enumerate(node.outputs):
            self.get_or_create_tensor(o, out_shapes[i] if i < len(out_shapes) else ())


class IGraphPass:
    """session.tkv:3630-3637."""

    def name(self) -> str:
        return ""

    def run(self, graph: ExecutionGraph) -> int:
        return 0


def _producers(graph: ExecutionGraph) -> Dict[str, ExecutionNode]:
    return {o: nd for nd in graph.nodes for o in nd.outputs}


def _consumers(graph: ExecutionGraph, name: str) -> int:
    return sum(1 for nd in graph.nodes for i in nd.inputs if i == name) + \
        sum(1 for o in graph.outputs if o == name)


def _float_const(graph: ExecutionGraph, name: str) -> Optional[np.ndarray]:
    return graph.initializers.get(name)


def _zero_point_is_zero(graph: ExecutionGraph, node: ExecutionNode) -> bool:
    """zp = int(first element) of input 2 (session.tkv:1905-1909); absent means 0.
    A zero point that is not a constant cannot be proven 0."""
    if len(node.inputs) < 3:
        return True
    zp = _float_const(graph, node.inputs[2])
    return zp is not None and zp.size > 0 and int(np.float32(zp[0])) == 0


def _axis(node: ExecutionNode, rank: int) -> int:
    return node.qlinear_axis if node.qlinear_axis >= 0 else node.qlinear_axis + rank


class QdqFoldPass(IGraphPass):
    """QdqFoldPass with quantized-GEMM emission (module docstring); ``emit_quantized_gemm``
    False gives the reference's drop-to-float behaviour alone."""

    def __init__(self, emit_quantized_gemm: bool = True):
        self.emit_quantized_gemm = emit_quantized_gemm

    def name(self) -> str:
        return "QdqFoldPass"

    def run(self, graph: ExecutionGraph) -> int:
        modified = 0
        if self.emit_quantized_gemm:
            modified |= self._fold_gemms(graph)
        modified |= self._drop_pairs(graph, keep_shared=self.emit_quantized_gemm)
        return modified

    # -- the reference's pass (session.tkv:3780-3805) --------------------------------------
    @staticmethod
    def _drop_pairs(graph: ExecutionGraph, keep_shared: bool = False) -> int:
        """With ``keep_shared``, a pair whose Q codes have another consumer (a folded
        QuantizedGemm) stays: the reference's loop would delete the Q under it."""
        modified = 0
        i = 0
        while i < len(graph.nodes):
            node = graph.nodes[i]
            if node.op_type == OperatorType_QuantizeLinear and len(node.outputs) == 1 and \
                    i + 1 < len(graph.nodes):
                nxt = graph.nodes[i + 1]
                if nxt.op_type == OperatorType_DequantizeLinear and len(nxt.inputs) > 0 and \
                        nxt.inputs[0] == node.outputs[0] and len(nxt.outputs) == 1 and \
                        not (keep_shared and _consumers(graph, node.outputs[0]) > 1):
                    orig, dead = node.inputs[0], nxt.outputs[0]
                    for nd in graph.nodes:
                        nd.inputs = [orig if t == dead else t for t in nd.inputs]
                    graph.outputs = [orig if t == dead else t for t in graph.outputs]
                    del graph.nodes[i + 1]
                    del graph.nodes[i]
                    modified = 1
                    continue
            i += 1
        return modified

    # -- the quantized-GEMM fold -------------------------------------------------------------
    def _fold_gemms(self, graph: ExecutionGraph) -> int:
        modified = 0
        i = 0
        while i < len(graph.nodes):
            nd = graph.nodes[i]
            folded = self._try_fold(graph, i) if nd.op_type in (
                OperatorType_MatMul, OperatorType_FusedLinear, OperatorType_Gemm) else None
            if folded is not None:
                modified = 1
                i = graph.nodes.index(folded) + 1
            else:
                i += 1
        return modified

    def _try_fold(self, graph: ExecutionGraph, idx: int) -> Optional[ExecutionNode]:
        mm = graph.nodes[idx]
        if len(mm.inputs) < 2 or len(mm.outputs) != 1:
            return None
        if mm.op_type == OperatorType_FusedLinear and mm.activation != ActivationFunction_None:
            return None
        if mm.op_type == OperatorType_Gemm and (np.float32(mm.alpha) != 1 or mm.trans_a != 0 or (
                len(mm.inputs) > 2 and np.float32(mm.beta) != 1)):
            return None
        prod = _producers(graph)
        dqa, dqw = prod.get(mm.inputs[0]), prod.get(mm.inputs[1])
        if dqa is None or dqw is None or dqa.op_type != OperatorType_DequantizeLinear or \
                dqw.op_type != OperatorType_DequantizeLinear:
            return None
        qa = prod.get(dqa.inputs[0])
        if qa is None or qa.op_type != OperatorType_QuantizeLinear or len(qa.outputs) != 1:
            return None
        # the DQ zero points define the values (a Q's zero point is already in its codes)
        if not (_zero_point_is_zero(graph, dqa) and _zero_point_is_zero(graph, dqw)):
            return None
        a_shape = graph.tensors[mm.inputs[0]].shape
        b_shape = graph.tensors[mm.inputs[1]].shape
        if len(a_shape) != 2 or len(b_shape) != 2:
            return None
        m, k = a_shape
        sa = _float_const(graph, dqa.inputs[1])
        sw = _float_const(graph, dqw.inputs[1])
        if sa is None or sa.size != 1 or sw is None:
            return None
        # B's layout as the reference's node reads it
        if mm.op_type == OperatorType_Gemm:
            b_nk = mm.trans_b != 0
            if b_shape[1 if b_nk else 0] != k:
                return None
            if b_nk and b_shape[0] != b_shape[1]:
                return None  # the reference's trans_b indexing (see the module docstring)
        elif b_shape[1] == k:
            b_nk = True
        elif b_shape[0] == k:
            b_nk = False
        else:
            return None
        n = b_shape[0] if b_nk else b_shape[1]
        if sw.size != 1 and (sw.size != n or _axis(dqw, 2) != (0 if b_nk else 1)):
            return None
        bias = None
        if len(mm.inputs) > 2:
            bias = mm.inputs[2]
            bd = graph.tensors.get(bias)
            if bd is None or _count(bd.shape) != n:
                return None
        # the weight codes: an int8 initializer, or Q of a float initializer
        wsrc = dqw.inputs[0]
        qw = None
        if wsrc in graph.initializers_int8:
            codes = graph.initializers_int8[wsrc]
        else:
            qw = prod.get(wsrc)
            if qw is None or qw.op_type != OperatorType_QuantizeLinear or \
                    any(t not in graph.initializers for t in qw.inputs):
                return None
            qin = [(graph.initializers[t], graph.tensors[t].shape) for t in qw.inputs]
            codes = qw.execute(qin, [b_shape])[0]
        if codes.size != n * k:
            return None
        if not b_nk:
            codes = np.ascontiguousarray(codes.reshape(k, n).T)
        wname = f"{mm.name}.qweight"
        while wname in graph.tensors:
            wname += "_"
        graph.add_initializer_int8(wname, codes, [n, k])

        q = new_node(mm.name, OperatorType_QuantizedGemm,
                     [qa.outputs[0], wname] + ([bias] if bias is not None else []), mm.outputs)
        q.scale_a = np.float32(sa[0])
        if sw.size == 1:
            q.scale_b = np.float32(sw[0])
        else:
            q.scales_w = [float(v) for v in sw]
        graph.nodes[idx] = q
        # DQ / Q nodes left without consumers go; the activation Q stays
        for dead in (dqa, dqw, qw):
            if dead is not None and dead in graph.nodes and \
                    all(_consumers(graph, o) == 0 for o in dead.outputs):
                graph.nodes.remove(dead)
        return q


def run_graph(graph: ExecutionGraph, feeds: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
    """Run a graph whose nodes are all quantized ops (session.py's QuantNode dispatch) in node
    order and return its outputs.  Float ops stay with the rest of the runtime: a graph that
    holds one raises before any node runs."""
    values: Dict[str, np.ndarray] = {}
    for name, v in feeds.items():
        values[name] = np.asarray(v)

    def fetch(name):
        if name in values:
            return values[name]
        if name in graph.initializers_int8:
            return graph.initializers_int8[name]
        if name in graph.initializers:
            return graph.initializers[name]
        raise KeyError(f"tensor {name!r} has no value")

    for nd in graph.nodes:
        if nd.op_type not in _QUANT_OPS:
            raise NotImplementedError(f"node {nd.name!r} (op {nd.op_type}) is not a quantized op")
    for nd in graph.nodes:
        ins = [(fetch(t), graph.tensors[t].shape) for t in nd.inputs]
        outs = nd.execute(ins, [graph.tensors[o].shape for o in nd.outputs])
        for o, v in zip(nd.outputs, outs):
            values[o] = v
    return {o: fetch(o) for o in graph.outputs}
