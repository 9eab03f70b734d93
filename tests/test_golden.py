"""The CPU oracle against the committed golden fixtures (tests/golden/).

* reference_kats.json holds the reference's own known-answer tests for this
  path. Each is checked here with the assert the reference uses.
* e4m3_decode.json and w8a8_pipeline.json were written by
  tests/golden/make_golden.py. Recomputing them here keeps the oracle from
  drifting under the digests that the GPU tests compare the HIP path with.
"""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


KATS = _load("reference_kats.json")


def test_kat_calibrate_minmax():
    kat = KATS["calibrate_minmax"]
    p = O.calibrate_minmax(np.array(kat["data"], np.float32), kat["symmetric"])
    assert abs(float(p.scale) - kat["scale"]) < kat["scale_abs_tol"]
    assert p.zero_point == kat["zero_point"]


def test_kat_quantize_roundtrip():
    kat = KATS["quantize_roundtrip"]
    x = np.array(kat["data"], np.float32)
    p = O.calibrate_minmax(x, kat["symmetric"])
    dq = O.dequantize_int8_symmetric(O.quantize_int8_symmetric(x, p.scale), p.scale)
    assert float(np.max(np.abs(x - dq))) <= float(p.scale) + 0.000001


@pytest.mark.parametrize("name,enc,dec", [
    ("fp8_e4m3_roundtrip", O.fp8_e4m3_encode, O.fp8_e4m3_decode),
    ("fp8_e5m2_roundtrip", O.fp8_e5m2_encode, O.fp8_e5m2_decode),
])
def test_kat_fp8_roundtrip(name, enc, dec):
    kat = KATS[name]
    for v in kat["data"]:
        v32 = float(np.float32(v))
        rec = float(dec(enc(v32)))
        assert abs(v32 - rec) / (abs(v32) + kat["den_eps"]) < kat["rel_tol"], v


def test_kat_matmul_integer():
    kat = KATS["matmul_integer"]
    y = O.matmul_integer(kat["a"], kat["b"], kat["m"] * kat["n"], kat["m"], kat["n"], kat["k"])
    assert list(y) == kat["y"]


def test_kat_dynamic_quantize_linear():
    kat = KATS["dynamic_quantize_linear"]
    y, ys, yz = O.dynamic_quantize_linear(kat["x"])
    assert abs(float(ys) - kat["y_scale"]) < kat["y_scale_abs_tol"]
    assert float(yz) == kat["y_zero_point"]
    for i, v in kat["y_index"].items():
        assert y[int(i)] == v


def test_e4m3_decode_table():
    table = _load("e4m3_decode.json")["f32_bits"]
    got = ["%08x" % int(np.float32(O.fp8_e4m3_decode(c)).view(np.uint32)) for c in range(256)]
    assert got == table


PIPE = _load("w8a8_pipeline.json")


@pytest.mark.parametrize("case", PIPE["cases"], ids=[c["name"] for c in PIPE["cases"]])
def test_w8a8_pipeline_digests(case):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden",
                                                  os.path.join(GOLDEN, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    s = case["seeds"]
    got = mg._case(case["name"], case["m"], case["n"], case["k"], s["x"], s["w"], s["bias"])
    assert got == case
