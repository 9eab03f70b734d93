"""QdqFoldPass rewrite rules on the CPU (no device work: the weights are int8 initializers).

The quantized-GEMM fold turns QDQ pairs in front of MatMul / FusedLinear / Gemm into the
reference's QuantizedGemm node (tv/runtime/session.tkv:678-697); what it cannot fold keeps
the reference's drop-to-float behaviour (session.tkv:3774-3805).  Numerics are in
tests/test_gpu_qdq_fold.py.
"""
import numpy as np
import pytest

from qdq_graphs import build, ops
from tokenvector.inference_amd import graph as G

Q, DQ, QG = G.OperatorType_QuantizeLinear, G.OperatorType_DequantizeLinear, \
    G.OperatorType_QuantizedGemm


def _qgemm(g):
    [q] = [nd for nd in g.nodes if nd.op_type == QG]
    return q


def test_matmul_kn_per_channel_folds_and_transposes():
    m, k, n = 4, 24, 10
    g, d = build(m, k, n, weight="int8")
    codes_kn = g.initializers_int8["Wc"].reshape(k, n)
    assert G.QdqFoldPass().run(g) == 1
    assert ops(g) == [Q, QG]
    q = _qgemm(g)
    assert q.inputs[0] == "x_q" and q.outputs == ["y"] and len(q.inputs) == 2
    wname = q.inputs[1]
    assert g.tensors[wname].shape == [n, k]
    assert np.array_equal(g.initializers_int8[wname], codes_kn.T.reshape(-1))
    assert np.float32(q.scale_a) == d["sx"]
    assert np.array_equal(np.array(q.scales_w, np.float32), d["sw"])
    # the activation Q node is the original one, untouched
    assert g.nodes[0].name == "qx" and g.nodes[0].inputs[:2] == ["x", "sx"]


def test_gemm_trans_b_with_bias_keeps_layout():
    # square B: the reference's Gemm (session.tkv:812-868) reads it as [N, K] under trans_b
    m, k, n = 3, 16, 16
    g, d = build(m, k, n, op=G.OperatorType_Gemm, b_nk=True, weight="int8", bias=True)
    codes = g.initializers_int8["Wc"].copy()
    assert G.QdqFoldPass().run(g) == 1
    q = _qgemm(g)
    assert q.inputs[2] == "bias"
    assert np.array_equal(g.initializers_int8[q.inputs[1]], codes)


def test_gemm_trans_b_non_square_is_not_folded():
    # _exec_gemm takes N from B.shape[1] and reads b[j * B.shape[0] + p] under trans_b, which
    # is not the [N, K] product for a non-square B: the node stays the reference's own
    m, k, n = 3, 16, 8
    g, d = build(m, k, n, op=G.OperatorType_Gemm, b_nk=True, weight="int8", bias=True)
    G.QdqFoldPass().run(g)
    assert not any(nd.op_type == G.OperatorType_QuantizedGemm for nd in g.nodes)
    assert any(nd.op_type == G.OperatorType_Gemm for nd in g.nodes)


def test_per_tensor_weight_scale_uses_scale_b():
    g, d = build(2, 8, 6, weight="int8", w_scale="tensor")
    G.QdqFoldPass().run(g)
    q = _qgemm(g)
    assert q.scales_w == [] and np.float32(q.scale_b) == d["sw"][0]


def test_square_matmul_reads_b_as_nk():
    # _exec_linear (session.tkv:756-762) checks B's second dimension against K first, so a
    # square B is [N, K]: its codes fold untransposed
    g, _ = build(2, 8, 8, weight="int8", b_nk=True)
    codes = g.initializers_int8["Wc"].copy()
    G.QdqFoldPass().run(g)
    assert np.array_equal(g.initializers_int8[_qgemm(g).inputs[1]], codes)


def test_fused_linear_without_activation_folds():
    g, _ = build(2, 8, 6, op=G.OperatorType_FusedLinear, weight="int8", bias=True)
    G.QdqFoldPass().run(g)
    assert ops(g) == [Q, QG]


@pytest.mark.parametrize("kw", [
    dict(act_dq_zp=3.0),                       # activation zero point
    dict(w_dq_zp=1.0),                         # weight zero point
    dict(w_axis=0),                            # per-channel scales on K, not N
    dict(op=G.OperatorType_Gemm, alpha=0.5),   # scaled product
    dict(op=G.OperatorType_Gemm, trans_a=1),
    dict(op=G.OperatorType_Gemm, bias=True, beta=2.0),
    dict(op=G.OperatorType_FusedLinear, activation=1),  # ReLU
])
def test_unfoldable_keeps_reference_behaviour(kw):
    g, _ = build(2, 8, 6, weight="int8", **kw)
    ref, _ = build(2, 8, 6, weight="int8", **kw)
    G.QdqFoldPass().run(g)
    G.QdqFoldPass(emit_quantized_gemm=False).run(ref)
    assert QG not in ops(g)
    assert ops(g) == ops(ref) and [nd.inputs for nd in g.nodes] == [nd.inputs for nd in ref.nodes]
    # the reference drops the adjacent activation pair: the product reads x in float
    mm = g.nodes[-1]
    assert mm.inputs[0] == "x"


def test_nonzero_activation_q_zero_point_still_folds():
    # the DQ's zero point defines the value; a Q's zero point is already in its codes
    g, _ = build(2, 8, 6, weight="int8", act_q_zp=2.0)
    G.QdqFoldPass().run(g)
    assert ops(g) == [Q, QG]


def test_reference_pass_alone_drops_to_float():
    g, _ = build(2, 8, 6, weight="float")
    assert G.QdqFoldPass(emit_quantized_gemm=False).run(g) == 1
    assert ops(g) == [G.OperatorType_MatMul]
    assert g.nodes[0].inputs == ["x", "W"]


def test_shared_dequantized_activation_stays():
    g, _ = build(2, 8, 6, weight="int8", dq_extra_consumer=True)
    G.QdqFoldPass().run(g)
    # the DQ output is a graph output, so DQ stays, and its Q (whose codes feed the folded
    # node) is not dropped under it
    assert ops(g) == [Q, DQ, QG]
    assert g.outputs == ["y", "x_dq"]


def test_run_graph_refuses_float_ops():
    g, d = build(2, 8, 6, weight="int8", act_dq_zp=3.0)
    G.QdqFoldPass().run(g)
    with pytest.raises(NotImplementedError):
        G.run_graph(g, {"x": d["x"]})
