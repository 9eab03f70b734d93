"""tokenvector.inference_amd -- MI355X (gfx950) implementation of
TokenVector.Inference's post-training-quantization hot path.

Submodules:
    quantization  mirror of tv/quantization/{engine,matmul}.tkv (host lists)
    session       mirror of the quantized nodes of tv/runtime/session.tkv
    graph         QdqFoldPass emitting the QuantizedGemm node, and a runner
                  for graphs of quantized nodes
    device        device-pointer API: contexts, buffers, packed kernels,
                  resident quantized weights and the W8A8 linear
    _lib          ctypes binding of libtkv_hip.so (C ABI in include/tkv_hip.h)
"""
from . import _lib

build = _lib.build


def device_count() -> int:
    return int(_lib.lib().tkv_hip_device_count())


__all__ = ["build", "device_count"]
