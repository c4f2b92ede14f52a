"""ingot_amd: MI355X (gfx950) backend for Ingot's MoE-layer hot path.

Routing, token-to-expert dispatch, grouped gate/up/SwiGLU/down expert products
on GGUF-quantized weights and the weighted combine, as hand-written HIP
kernels behind a C ABI (include/ingot_moe.h, ingot_amd/libingot_moe.so).
"""
from .moe import (DeviceError, Gpu, InvalidData, LayerSpec, Matrix, MoeLayer, NonFinite, Unsupported,  # noqa: F401
                  geometry, route)

__all__ = ["DeviceError", "Gpu", "InvalidData", "LayerSpec", "Matrix", "MoeLayer", "NonFinite", "Unsupported",
           "geometry", "route"]
