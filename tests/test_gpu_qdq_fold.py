"""QdqFoldPass's QuantizedGemm on the GPU.

The folded graph (activation Q + QuantizedGemm, tv/runtime/session.tkv:678-697) must equal the
reference's own node chain run by the oracle bit for bit: the Q codes of x and of the weight,
then ``quantized_gemm_node`` on them.  Against the float path it replaces (the dequantized
operands multiplied in f32), the stated tolerance is
    |y_fold - y_float| <= 2^-24 |y_fold| + (K + 4) 2^-24 (sum_k |dqx_k| |dqw_k| + |b|),
and against the unquantized product x W^T + b the quantization bound
    |y_fold - y_true| <= sum_k (ex_k |w_k| + |dqx_k| ew_k) + the float-path term above,
with ex = sx / 2 (1 + 2^-20) + 2^-23 |x| and ew = sw[n] / 2 (1 + 2^-20) + 2^-23 |w| (half a
quantization step, the rounding of the quotient before it and of the dequantized value).
"""
import numpy as np
import pytest

import oracle as O
from qdq_graphs import build, ops
from tokenvector.inference_amd import graph as G

pytestmark = pytest.mark.gpu

U = 2.0 ** -24

CASES = {
    # qkv-shaped MatMul, B = [K, N], float weights quantized by the fold, per-channel scales
    "matmul_kn_float_w": dict(m=64, k=768, n=2304),
    # attn_out-shaped Gemm with trans_b (a square B, which the reference reads as [N, K])
    # and a bias
    "gemm_nk_bias": dict(m=200, k=768, n=768, op=G.OperatorType_Gemm, b_nk=True, bias=True),
    # FusedLinear on stored int8 codes with one weight scale
    "fused_int8_w_tensor_scale": dict(m=33, k=256, n=96, op=G.OperatorType_FusedLinear,
                                      weight="int8", w_scale="tensor", bias=True),
    # one token, ragged N
    "matmul_m1_ragged": dict(m=1, k=64, n=40, b_nk=True),
}


def _oracle_codes(g, d, case):
    """The Q node's codes per the oracle: x per tensor, the weight on B's layout."""
    m, k, n = case["m"], case["k"], case["n"]
    b_nk = case.get("b_nk", False)
    qx = O.quantize_linear(d["x"], [d["sx"]])
    if case.get("weight", "float") == "float":
        B = g.initializers["W"]
        if d["sw"].size == 1:
            qb = O.quantize_linear(B, d["sw"])
        elif b_nk:
            qb = O.quantize_linear(B, d["sw"], 0, 1, n, k)
        else:
            qb = O.quantize_linear(B, d["sw"], 0, k, n, 1)
    else:
        qb = g.initializers_int8["Wc"]
    wnk = qb.reshape(n, k) if b_nk else qb.reshape(k, n).T
    return qx, np.ascontiguousarray(wnk).reshape(-1)


@pytest.mark.parametrize("name", list(CASES))
def test_folded_graph_matches_reference_nodes_and_float_path(hip, name):
    case = CASES[name]
    m, k, n = case["m"], case["k"], case["n"]
    extra = {kk: v for kk, v in case.items() if kk not in ("m", "k", "n")}
    g, d = build(m, k, n, seed=7, **extra)
    qx, wnk = _oracle_codes(g, d, case)
    assert G.QdqFoldPass().run(g) == 1
    assert ops(g) == [G.OperatorType_QuantizeLinear, G.OperatorType_QuantizedGemm]
    q = g.nodes[1]
    # the weight codes the fold produced on the GPU equal the oracle's Q
    assert np.array_equal(g.initializers_int8[q.inputs[1]], wnk)

    y = G.run_graph(g, {"x": d["x"]})["y"]
    assert y.dtype == np.float32 and y.size == m * n

    # 1. bit-exact against the reference's node chain
    b = d["b"]
    sws = d["sw"] if d["sw"].size > 1 else None
    want = O.quantized_gemm_node(qx, wnk, b, m, n, k, d["sx"],
                                 d["sw"][0] if sws is None else 1.0, sws)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))

    # 2. the float path: dequantized operands (one f32 rounding each), f32 product
    sw_n = np.broadcast_to(d["sw"], (n,)).astype(np.float32)
    dqx = (qx.astype(np.float32) * d["sx"]).reshape(m, k)
    dqw = (wnk.astype(np.float32).reshape(n, k) * sw_n[:, None]).astype(np.float32)
    bf = b if b is not None else np.zeros(n, np.float32)
    y_float = (dqx @ dqw.T + bf).astype(np.float32)
    terms = np.abs(dqx).astype(np.float64) @ np.abs(dqw).astype(np.float64).T + np.abs(bf)
    yy = y.reshape(m, n).astype(np.float64)
    bound = U * np.abs(yy) + (k + 4) * U * terms
    err = np.abs(yy - y_float.astype(np.float64))
    assert np.all(err <= bound), (name, float((err / bound).max()))

    # 3. the quantization bound against the unquantized product
    x64, w64 = d["x"].astype(np.float64), d["w"].astype(np.float64)
    y_true = x64 @ w64.T + bf
    ex = d["sx"] / 2 * (1 + 2.0 ** -20) + 2.0 ** -23 * np.abs(x64)
    ew = sw_n[:, None] / 2 * (1 + 2.0 ** -20) + 2.0 ** -23 * np.abs(w64)
    qbound = ex @ np.abs(w64).T + np.abs(dqx) @ ew.T + bound
    assert np.all(np.abs(yy - y_true) <= qbound), name


def test_shared_dequantized_activation_runs(hip):
    m, k, n = 16, 128, 48
    g, d = build(m, k, n, seed=3, weight="int8", dq_extra_consumer=True)
    G.QdqFoldPass().run(g)
    out = G.run_graph(g, {"x": d["x"]})
    qx = O.quantize_linear(d["x"], [d["sx"]])
    assert np.array_equal(out["x_dq"], O.dequantize_linear(qx, [d["sx"]]))
    wnk = g.initializers_int8[g.nodes[-1].inputs[1]]
    want = O.quantized_gemm_node(qx, wnk, None, m, n, k, d["sx"], 1.0, d["sw"])
    assert np.array_equal(out["y"].view(np.uint32), want.view(np.uint32))
