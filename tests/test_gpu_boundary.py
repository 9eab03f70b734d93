"""The C ABI's fallback and re-entrancy contract on a real device.

* rc -1 (TKV_HIP_UNSUPPORTED, the .tkv caller keeps its own loop,
  docs/HANDOFF.md:3649) for what the INT32 datapath cannot express: K >= 2^17
  (|acc| could pass 2^31) and codes outside the int8 range in the reference's
  int32 code lists.
* Re-entrancy: two host threads driving host mirrors at the same time, each
  on its own default context, give the single-threaded results bit for bit
  (the reference's shared-job native library hung two callers,
  docs/COMPILER_TEAM_REQUEST2.md:46,91).
"""
import ctypes as C
import sys
import threading

import numpy as np
import pytest

import oracle as O
from tokenvector.inference_amd import _lib
from tokenvector.inference_amd import device as D
from tokenvector.inference_amd import quantization as Q

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def test_unsupported_k_and_codes(hip):
    say("rc -1: K >= 2^17, codes outside int8")
    L = _lib.lib()
    ctx = D.Context(0)
    k = 1 << 17
    da = D.DeviceBuffer.empty(ctx, k, np.int8)
    dw = D.DeviceBuffer.empty(ctx, k, np.int8)
    dacc = D.DeviceBuffer.empty(ctx, 1, np.int32)
    rc = L.tkv_hip_dev_matmul_int8_accum(ctx.handle, C.c_void_p(da.ptr), C.c_void_p(dw.ptr), 1, 1,
                                         k, C.c_void_p(dacc.ptr))
    assert rc == _lib.UNSUPPORTED
    # the same K through a host mirror
    a = np.ones(k, np.int32)
    acc = np.zeros(1, np.int32)
    assert L.tkv_hip_matmul_int8_accum(_p(a), _p(a), _p(acc), 1, 1, k) == _lib.UNSUPPORTED
    # K just below the limit runs and is exact (the mirror zero pads its
    # rows to 2^17 bytes; the bound is on the caller's K)
    a = np.full(k - 1, -128, np.int32)
    assert L.tkv_hip_matmul_int8_accum(_p(a), _p(a), _p(acc), 1, 1, k - 1) == _lib.OK
    assert int(acc[0]) == 128 * 128 * (k - 1)
    # int32 codes that do not fit the int8 datapath
    m, n, kk = 4, 5, 64
    a = np.zeros(m * kk, np.int32)
    a[7] = 200
    w = np.ones(n * kk, np.int32)
    y = np.zeros(m * n, np.float32)
    rc = L.tkv_hip_matmul_int8_symmetric(_p(a), _p(w), None, 0, _p(y), m, n, kk, C.c_float(1.0),
                                         C.c_float(1.0))
    assert rc == _lib.UNSUPPORTED
    a[7] = -129
    rc = L.tkv_hip_matmul_int8_symmetric(_p(a), _p(w), None, 0, _p(y), m, n, kk, C.c_float(1.0),
                                         C.c_float(1.0))
    assert rc == _lib.UNSUPPORTED
    for b in (da, dw, dacc):
        b.close()
    ctx.close()


def test_two_threads_drive_host_mirrors(hip):
    """Calibrate + quantize + INT8 GEMM through the host mirrors from two
    threads at once (ctypes releases the GIL during each call), repeatedly;
    every result equals the oracle's."""
    say("two threads on host mirrors")
    m, n, k = 96, 160, 768
    cases = []
    for t in range(2):
        x = O.gi_noise(m * k, 100 + t, 1.0)
        w = O.gi_noise(n * k, 200 + t, 0.02)
        b = O.gi_noise(n, 300 + t, 0.01)
        osw = np.array([p.scale for p in O.calibrate_per_channel_minmax(w, n, k)], np.float32)
        owq = O.quantize_int8_per_channel(w, n, k, osw)
        opx = O.calibrate_minmax(x, 1)
        oxq = O.quantize_int8_symmetric(x, opx.scale)
        oy = O.matmul_int8_per_channel(oxq, owq, b, m, n, k, opx.scale, osw)
        cases.append((x, w, b, oy))
    errors = []
    start = threading.Barrier(2)

    def run(t):
        x, w, b, oy = cases[t]
        try:
            start.wait()
            for it in range(20):
                sw = np.array([p.scale for p in Q.calibrate_per_channel_minmax(w, n, k)], np.float32)
                wq = np.zeros(n * k, np.int32)
                Q.quantize_int8_per_channel(w, wq, n, k, sw)
                px = Q.calibrate_minmax(x, 1)
                xq = np.zeros(m * k, np.int32)
                Q.quantize_int8_symmetric(x, xq, px.scale)
                y = np.zeros(m * n, np.float32)
                Q.matmul_int8_per_channel(xq, wq, b, y, m, n, k, px.scale, sw)
                if not np.array_equal(y.view(np.uint32), oy.view(np.uint32)):
                    errors.append((t, it))
                    return
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append((t, repr(e)))

    th = [threading.Thread(target=run, args=(t,)) for t in range(2)]
    for h in th:
        h.start()
    for h in th:
        h.join(timeout=100)
    assert not any(h.is_alive() for h in th), "a mirror call did not return"
    assert not errors, errors


def test_context_destroyed_before_its_graph(hip):
    """A context closed while one of its graphs is alive releases the graph's
    executable and detaches it: launching it later is TKV_HIP_BAD_ARG, and
    destroying it afterwards frees only the handle (the order of the two
    destructions no longer matters)."""
    say("context closed before its graph")
    L = _lib.lib()
    ctx = D.Context(0)
    n = 4096
    dx = D.DeviceBuffer.from_host(ctx, O.gi_noise(n, 3, 1.0))
    dq = D.DeviceBuffer.empty(ctx, n, np.int8)
    p = D.params_buffer(ctx)
    D.quantize_int8_dynamic_tensor(ctx, dx, n, dq, p)
    ctx.synchronize()
    with D.Graph(ctx) as g:
        D.quantize_int8_dynamic_tensor(ctx, dx, n, dq, p)
    g.launch()
    ctx.synchronize()
    handle = g.handle
    for buf in (dx, dq, p):
        buf.close()
    ctx.close()                                   # before the graph
    other = D.Context(0)
    assert L.tkv_hip_graph_launch(other.handle, handle) == _lib.BAD_ARG
    g.close()                                     # detached: frees the handle only
    assert g.handle == 0
    other.close()


def test_set_tuning_ranges(hip):
    """Per-context tuning overrides: each knob accepts its documented range
    and -1, and refuses anything else (and unknown knobs) with BAD_ARG."""
    L = _lib.lib()
    ctx = D.Context(0)
    ranges = {D.TUNE_GEMM_CFG: (0, 11), D.TUNE_GEMM_STAGGER: (0, 8),
              D.TUNE_DECODE_GROUP: (1, 16), D.TUNE_QUANT_TWO_PASS: (0, 1),
              D.TUNE_INT4_GEMV_WAVE: (0, 1), D.TUNE_GRID_SPIN: (0, 1 << 20),
              D.TUNE_DECODE_DMA: (0, 1)}
    for knob, (lo, hi) in ranges.items():
        for v in (lo, hi, -1):
            assert L.tkv_hip_ctx_set_tuning(ctx.handle, knob, v) == _lib.OK, (knob, v)
        for v in (lo - 1 if lo - 1 != -1 else -2, hi + 1):
            assert L.tkv_hip_ctx_set_tuning(ctx.handle, knob, v) == _lib.BAD_ARG, (knob, v)
    assert L.tkv_hip_ctx_set_tuning(ctx.handle, 7, 0) == _lib.BAD_ARG
    assert L.tkv_hip_ctx_set_tuning(ctx.handle, -1, 0) == _lib.BAD_ARG
    ctx.close()
