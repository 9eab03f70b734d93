"""Writes the golden fixtures under tests/golden/.

    python tests/golden/make_golden.py            # rewrite every fixture
    python tests/golden/make_golden.py --check    # recompute, compare, write nothing

Fixtures (all data, no code):

* ``reference_kats.json``: the known-answer vectors of the reference's own
  tests for this path, transcribed with their file:line. These are inputs,
  expected outputs and the tolerance each assert uses.
* ``e4m3_decode.json``: the f32 bit pattern each of the 256 e4m3 codes
  decodes to under the reference decoder (tv/quantization/types.tkv:193-233).
* ``w8a8_pipeline.json``: SHA-256 digests of every stage of the W8A8
  pipeline at full size on the seeded inputs of the benchmark workloads:
  config 1 (X [1024,768], W [3072,768]) and the four GPT-2-124M linears at
  M = 8192. The stages are weight per-channel scales and codes, activation
  per-tensor scale and codes, per-row scales and codes, and the dequantized
  outputs for both activation modes. The GPU tests compare the HIP path with
  these digests bit for bit, without recomputing a GEMM on the host.

The digests come from the CPU oracle (oracle/tkv_oracle.c) for the
quantization stages and from an exact float64 BLAS product for the INT32
accumulators. |acc| <= 127^2 * 3072 < 2^53, so the float64 product is exact.
The per-tensor outputs are additionally cross-checked against the oracle's
own GEMM.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402

# Seeds of tv/training/gpt2_ref.tkv's LCG31 + Box-Muller generator, as used by
# bench.py (activations by K, weights and biases by linear index).
GPT2_LINEARS = [("qkv", 2304, 768), ("attn_out", 768, 768), ("mlp_up", 3072, 768),
                ("mlp_down", 768, 3072)]
X_SEED = {768: 0, 3072: 7}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def f32_hex(v) -> str:
    return "%08x" % int(np.float32(v).view(np.uint32))


def reference_kats() -> dict:
    return {
        "calibrate_minmax": {
            "source": "tv/tests/gap_tests.tkv:158-168",
            "data": [-12.7, 0.0, 6.35, 12.7], "symmetric": 1,
            "scale": 0.1, "scale_abs_tol": 0.00001, "zero_point": 0,
        },
        "quantize_roundtrip": {
            "source": "tv/tests/gap_tests.tkv:171-193",
            "data": [-1.5, -0.5, 0.0, 0.5, 1.5], "symmetric": 1,
            "rule": "max|x - dequantize(quantize(x, s), s)| <= s + 0.000001, s = calibrate(x).scale",
        },
        "fp8_e4m3_roundtrip": {
            "source": "tv/tests/gap_tests.tkv:196-218",
            "data": [0.0, 0.5, 1.0, -1.0, 2.5, 16.0], "rel_tol": 0.15, "den_eps": 0.00001,
        },
        "fp8_e5m2_roundtrip": {
            "source": "tv/tests/gap_tests.tkv:219-240",
            "data": [0.0, 0.25, 1.0, -2.0, 64.0, 512.0], "rel_tol": 0.25, "den_eps": 0.00001,
        },
        "matmul_integer": {
            "source": "tv/tests/inference_tests.tkv:896-922",
            "a": [1, 2, 3, 4], "b": [1, 1, 1, 1], "m": 2, "n": 2, "k": 2, "y": [3, 3, 7, 7],
        },
        "dynamic_quantize_linear": {
            "source": "tv/tests/inference_tests.tkv:923-948",
            "x": [0.0, 1.0, 2.0], "y_scale": 2.0 / 255.0, "y_scale_abs_tol": 0.000001,
            "y_zero_point": 0.0, "y_index": {"0": -128, "2": 127},
        },
    }


def e4m3_decode_table() -> dict:
    return {
        "source": "tv/quantization/types.tkv:193-233 (decoder), oracle tkvo_fp8_e4m3_decode",
        "f32_bits": [f32_hex(O.fp8_e4m3_decode(c)) for c in range(256)],
    }


def _case(name: str, m: int, n: int, k: int, x_seed: int, w_seed: int, b_seed: int) -> dict:
    x = O.gi_noise(m * k, x_seed, 1.0)
    w = O.gi_noise(n * k, w_seed, 0.02)
    b = O.gi_noise(n, b_seed, 0.01)
    sw = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, n, k)], np.float32)
    wq = O.quantize_int8_per_channel(w, n, k, sw)
    px = O.calibrate_minmax(x, 1)
    xq = O.quantize_int8_symmetric(x, px.scale)
    xr, sr = O.quantize_dynamic_int8_rowwise(x, m, k)

    wf = wq.reshape(n, k).astype(np.float64)
    acc_t = xq.reshape(m, k).astype(np.float64) @ wf.T            # exact: |acc| < 2^53
    y_t = ((acc_t * np.float64(np.float32(px.scale))) * sw.astype(np.float64)[None, :]
           + b.astype(np.float64)[None, :]).astype(np.float32)
    y_o = O.matmul_int8_per_channel(xq, wq, b, m, n, k, px.scale, sw,
                                    threads=O.host_threads()).reshape(m, n)
    if not np.array_equal(y_t.view(np.uint32), y_o.view(np.uint32)):
        raise RuntimeError(f"{name}: oracle GEMM and exact product disagree")
    acc_r = xr.reshape(m, k).astype(np.float64) @ wf.T
    y_r = ((acc_r * sr.astype(np.float64)[:, None]) * sw.astype(np.float64)[None, :]
           + b.astype(np.float64)[None, :]).astype(np.float32)
    return {
        "name": name, "m": m, "n": n, "k": k,
        "seeds": {"x": x_seed, "w": w_seed, "bias": b_seed},
        "sigma": {"x": 1.0, "w": 0.02, "bias": 0.01},
        "w_scales_sha256": sha(sw), "w_codes_sha256": sha(wq.astype(np.int8)),
        "x_scale_f32": f32_hex(px.scale), "x_codes_sha256": sha(xq.astype(np.int8)),
        "x_row_scales_sha256": sha(sr), "x_row_codes_sha256": sha(xr.astype(np.int8)),
        "y_per_tensor_sha256": sha(y_t), "y_per_token_sha256": sha(y_r),
        "y_per_tensor_head_f32": [f32_hex(v) for v in y_t.reshape(-1)[:8]],
    }


def w8a8_pipeline() -> dict:
    cases = [_case("config1_mlp_up_m1024", 1024, 3072, 768, 0, 1, 2)]
    for j, (nm, n, k) in enumerate(GPT2_LINEARS):
        cases.append(_case(f"gpt2_{nm}_m8192", 8192, n, k, X_SEED[k], 11 + j, 61 + j))
    return {
        "generator": "oracle.gi_noise(n, seed, sigma) = tv/training/gpt2_ref.tkv LCG31 + Box-Muller",
        "pipeline": "W: calibrate_per_channel_minmax + quantize_int8_per_channel; "
                    "X per-tensor: calibrate_minmax(sym) + quantize_int8_symmetric; "
                    "X per-token: quantize_dynamic_int8_rowwise; "
                    "Y = f32(f64(f64(acc * s_a) * s_w[n]) + bias[n])",
        "cases": cases,
    }


FIXTURES = {
    "reference_kats.json": reference_kats,
    "e4m3_decode.json": e4m3_decode_table,
    "w8a8_pipeline.json": w8a8_pipeline,
}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true")
    args = ap.parse_args()
    bad = 0
    for fname, fn in FIXTURES.items():
        data = fn()
        path = os.path.join(HERE, fname)
        if args.check:
            with open(path) as f:
                same = json.load(f) == json.loads(json.dumps(data))
            print(f"{fname}: {'ok' if same else 'DIFFERS'}")
            bad += not same
        else:
            with open(path, "w") as f:
                json.dump(data, f, indent=1)
                f.write("\n")
            print(f"wrote {path}")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
