"""ctypes bindings of the two native libraries built in-tree.

* ``libingot_moe.so``  -- the HIP backend (include/ingot_moe.h). There is no
  Python or CPU fallback for anything it computes: if the library is missing
  or cannot be loaded, every entry point raises ``NativeLibraryMissing``.
* ``libingot_synth.so`` -- host-only synthetic inputs and GGUF-block
  quantizers (include/ingot_synth.h).
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
MOE_LIB = os.path.join(HERE, "libingot_moe.so")
# INGOT_SYNTH_LIB: another build of synth.cpp (the host sanitizer build of
# `make -C oracle sanitize`).
SYNTH_LIB = os.environ.get("INGOT_SYNTH_LIB") or os.path.join(HERE, "libingot_synth.so")


class NativeLibraryMissing(RuntimeError):
    pass


class Matrix_t(C.Structure):
    """struct ingot_matrix (include/ingot_moe.h)."""

    _fields_ = [
        ("data", C.c_void_p),
        ("nbytes", C.c_uint64),
        ("cols", C.c_uint64),
        ("rows", C.c_uint64),
        ("count", C.c_uint64),
        ("kind", C.c_uint32),
        ("stride", C.c_uint64),
    ]


class LayerDesc_t(C.Structure):
    """struct ingot_layer_desc (include/ingot_moe.h)."""

    _fields_ = [
        ("hidden", C.c_uint32),
        ("experts", C.c_uint32),
        ("top_k", C.c_uint32),
        ("routing", C.c_uint32),
        ("route_scale", C.c_float),
        ("swiglu_limit", C.c_float),
        ("router", C.c_void_p),
        ("router_bias", C.c_void_p),
        ("gate", Matrix_t),
        ("up", Matrix_t),
        ("down", Matrix_t),
        ("shared_gate", Matrix_t),
        ("shared_up", Matrix_t),
        ("shared_down", Matrix_t),
        ("shared_gate_vec", C.c_void_p),
        ("norm_gain", C.c_void_p),
        ("norm_eps", C.c_float),
    ]


P = C.c_void_p
U32 = C.c_uint32
U64 = C.c_uint64
I32 = C.c_int
F32 = C.c_float
PU32 = C.POINTER(C.c_uint32)
PF32 = C.POINTER(C.c_float)

# name -> (restype, argtypes): every symbol include/ingot_moe.h declares.
MOE_SYMBOLS = {
    "ingot_geometry": (I32, [U32, PU32, PU32]),
    "ingot_validate_matrix": (I32, [C.POINTER(Matrix_t)]),
    "ingot_status_string": (C.c_char_p, [I32]),
    "ingot_kind_supported": (I32, [U32]),
    "ingot_ctx_create": (I32, [I32, C.POINTER(P)]),
    "ingot_ctx_destroy": (I32, [P]),
    "ingot_last_error": (C.c_char_p, [P]),
    "ingot_ctx_set_stream": (I32, [P, P]),
    "ingot_ctx_stream": (P, [P]),
    "ingot_ctx_synchronize": (I32, [P]),
    "ingot_device_name": (C.c_char_p, [P]),
    "ingot_route": (I32, [P, P, U32, U32, P, P]),
    "ingot_project": (I32, [P, C.POINTER(Matrix_t), P, P]),
    "ingot_dequant": (I32, [P, C.POINTER(Matrix_t), P]),
    "ingot_moe": (I32, [P, C.POINTER(Matrix_t), C.POINTER(Matrix_t), C.POINTER(Matrix_t), P, P, U32, P]),
    "ingot_route_batch": (I32, [P, P, P, U32, U32, U32, U32, F32, P, P]),
    "ingot_ctx_check_device_flags": (I32, [P]),
    "ingot_layer_flag_status": (I32, [P]),
    "ingot_layer_create": (I32, [P, C.POINTER(LayerDesc_t), C.POINTER(P)]),
    "ingot_layer_clone": (I32, [P, C.POINTER(P)]),
    "ingot_layer_create_cached": (I32, [P, C.POINTER(LayerDesc_t), U32, C.POINTER(P)]),
    "ingot_layer_cache_stats": (I32, [P, C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)]),
    "ingot_expert_cache_create": (P, [U32]),
    "ingot_expert_cache_destroy": (None, [P]),
    "ingot_expert_cache_hit": (I32, [P, U32]),
    "ingot_expert_cache_claim": (I32, [P, U32, P, U32, C.POINTER(I32)]),
    "ingot_expert_cache_commit": (I32, [P, U32, U32]),
    "ingot_expert_cache_state": (I32, [P, P, C.POINTER(U64), C.POINTER(U64)]),
    "ingot_layer_destroy": (None, [P]),
    "ingot_layer_reserve": (I32, [P, U32]),
    "ingot_layer_forward": (I32, [P, P, U32, P, P, P]),
    "ingot_layer_forward_add": (I32, [P, P, P, U32, P, P, P]),
    "ingot_layer_forward_static": (I32, [P, P, U32, P, P, P]),
    "ingot_layer_static_bytes": (U64, [P, U32]),
    "ingot_layer_weight_bytes": (U64, [P]),
    "ingot_layer_set_gemm_mode": (I32, [P, U32]),
    "ingot_graph_begin": (I32, [P]),
    "ingot_graph_end": (I32, [P, C.POINTER(P)]),
    "ingot_graph_launch": (I32, [P, P]),
    "ingot_graph_destroy": (None, [P]),
    "ingot_graph_time": (I32, [P, P, U32, PF32]),
    "ingot_layer_time_stage": (I32, [P, U32, U32, PF32]),
    "ingot_layers_time_stage": (I32, [C.POINTER(P), U32, U32, U32, PF32]),
    "ingot_layer_stage_kernel": (C.c_char_p, [P, U32]),
    "ingot_layer_dispatch_debug": (I32, [P, P, P, P, P, P, U32, P]),
    "ingot_malloc": (I32, [P, U64, C.POINTER(P)]),
    "ingot_free": (I32, [P, P]),
    "ingot_memcpy_h2d": (I32, [P, P, P, U64]),
    "ingot_memcpy_d2h": (I32, [P, P, P, U64]),
    "ingot_device_mem_info": (I32, [P, C.POINTER(U64), C.POINTER(U64)]),
    "ingot_device_copy": (I32, [P, P, P, U64]),
    "ingot_device_read": (I32, [P, P, U64, P]),
}

SYNTH_SYMBOLS = {
    "ingot_synth_stream": (U64, [U64, U64, U64, U64]),
    "ingot_synth_normal": (None, [U64, U64, U64, F32, F32, P, I32]),
    "ingot_synth_uniform": (None, [U64, U64, U64, F32, F32, P, I32]),
    "ingot_round_bf16": (None, [P, U64]),
    "ingot_f32_to_f16": (C.c_uint16, [F32]),
    "ingot_f16_to_f32": (F32, [C.c_uint16]),
    "ingot_quant_row_bytes": (U64, [U32, U64]),
    "ingot_quantize": (I32, [U32, P, U64, U64, P, I32]),
    "ingot_synth_quantized": (I32, [U32, U64, U64, U64, U64, F32, P, I32]),
}

_cache: dict[str, C.CDLL] = {}


def _load(path: str, symbols: dict) -> C.CDLL:
    if path in _cache:
        return _cache[path]
    if not os.path.exists(path):
        raise NativeLibraryMissing(
            f"{os.path.basename(path)} is not built; run __graft_entry__.build() (or python -m ingot_amd.build)"
        )
    lib = C.CDLL(path)
    for name, (res, args) in symbols.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _cache[path] = lib
    return lib


def moe_lib() -> C.CDLL:
    return _load(MOE_LIB, MOE_SYMBOLS)


def synth_lib() -> C.CDLL:
    return _load(SYNTH_LIB, SYNTH_SYMBOLS)
