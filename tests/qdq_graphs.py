"""QDQ graphs around one MatMul / FusedLinear / Gemm, for the QdqFoldPass tests.

    [W -> Q(sw)] -> DQ(sw) ---\\
    x -> Q(sx) -> DQ(sx) ------> op (+ bias) -> y

The weight is either a float initializer behind a Q node (``weight="float"``) or int8 codes
stored as an initializer (``weight="int8"``; the codes come from numpy's rounding, any
in-range codes will do).  ``b_nk`` stores B as [N, K] (else [K, N]); ``w_scale`` is
"channel" (one scale per output column, on B's N axis unless ``w_axis`` says otherwise) or
"tensor".
"""
from __future__ import annotations

import numpy as np

from tokenvector.inference_amd import graph as G


def build(m, k, n, *, op=G.OperatorType_MatMul, b_nk=False, weight="float", w_scale="channel",
          w_axis=None, bias=False, act_dq_zp=None, act_q_zp=None, w_dq_zp=None, alpha=1.0,
          beta=1.0, trans_a=0, activation=0, dq_extra_consumer=False, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)  # logical [N, K]
    w[:, 0] *= 4.0  # spread the per-channel scales
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    sx = np.float32(np.abs(x).max() / 127.0)
    sw = (np.abs(w).max(axis=1) / 127.0).astype(np.float32) if w_scale == "channel" else \
        np.array([np.abs(w).max() / 127.0], np.float32)
    B = w if b_nk else np.ascontiguousarray(w.T)
    b_shape = [n, k] if b_nk else [k, n]
    axis = (0 if b_nk else 1) if w_axis is None else w_axis

    g = G.ExecutionGraph()
    g.inputs = ["x"]
    g.get_or_create_tensor("x", [m, k])
    g.add_initializer("sx", [sx], [1])
    g.add_initializer("sw", sw, [sw.size])

    def zp_input(name, v):
        if v is None:
            return []
        g.add_initializer(name, [v], [1])
        return [name]

    if weight == "float":
        g.add_initializer("W", B, b_shape)
        qw = G.new_node("qw", G.OperatorType_QuantizeLinear, ["W", "sw"], ["W_q"])
        qw.qlinear_axis = axis
        g.add_node(qw, [b_shape])
        wsrc = "W_q"
    else:
        sb = sw.reshape((-1, 1) if b_nk else (1, -1)) if sw.size > 1 else sw[0]
        codes = np.clip(np.rint(B / sb), -127, 127).astype(np.int32)
        g.add_initializer_int8("Wc", codes, b_shape)
        wsrc = "Wc"
    dqw = G.new_node("dqw", G.OperatorType_DequantizeLinear,
                     [wsrc, "sw"] + zp_input("zw", w_dq_zp), ["W_dq"])
    dqw.qlinear_axis = axis
    g.add_node(dqw, [b_shape])
    qx = G.new_node("qx", G.OperatorType_QuantizeLinear, ["x", "sx"] + zp_input("zxq", act_q_zp),
                    ["x_q"])
    g.add_node(qx, [[m, k]])
    dqx = G.new_node("dqx", G.OperatorType_DequantizeLinear,
                     ["x_q", "sx"] + zp_input("zx", act_dq_zp), ["x_dq"])
    g.add_node(dqx, [[m, k]])
    ins = ["x_dq", "W_dq"]
    if bias:
        g.add_initializer("bias", b, [n])
        ins.append("bias")
    mm = G.new_node("mm", op, ins, ["y"])
    mm.alpha, mm.beta = np.float32(alpha), np.float32(beta)
    mm.trans_a, mm.trans_b, mm.activation = trans_a, int(b_nk), activation
    g.add_node(mm, [[m, n]])
    g.outputs = ["y"] + (["x_dq"] if dq_extra_consumer else [])
    return g, dict(x=x, w=w, b=b if bias else None, sx=sx, sw=sw)


def ops(g):
    return [nd.op_type for nd in g.nodes]
