"""GGUF block formats feeding the quantized linears (tv/format/gguf.tkv:284-313),
decoded on libtkv_hip: the Q8_0, Q4_0 and Q4_1 branches of the reference's
``_dequant_tensor``.  Other dtypes raise (the reader keeps its own loop)."""
from __future__ import annotations

import numpy as np

from . import _lib
from .quantization import _p

GGUF_Q4_0 = 2
GGUF_Q4_1 = 3
GGUF_Q8_0 = 8


def dequant_blocks(raw, base: int, n: int, dtype: int) -> np.ndarray:
    """n elements of the tensor whose blocks start at raw[base] (the
    reference's ``out`` list: elements past the last whole block are 0)."""
    r = np.frombuffer(bytes(raw), np.uint8)[int(base):]
    r = np.ascontiguousarray(r) if r.size else np.zeros(1, np.uint8)
    out = np.zeros(max(int(n), 1), np.float32)
    _lib.check(_lib.lib().tkv_hip_dequantize_gguf(_p(r), r.size, int(n), int(dtype), _p(out),
                                                  out.size))
    return out[: int(n)]
