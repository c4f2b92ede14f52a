"""Synthetic MoE layers and inputs for the benchmark configurations.

Weights are drawn N(0, 0.02) and quantized by libingot_synth (this project's
own quantizers: Ingot only reads GGUF). Every tensor comes from its own
SplitMix64 stream keyed (config, layer, tensor, expert), so the CPU oracle and
the GPU consume identical bytes on any machine and thread count.

    C0  Qwen3-30B-A3B-shaped layer, decode 1 token: H 2048, E 128, top-8
        softmax, F 768, Q4_K experts, fp32 router [128 x 2048]
    C1  C0's layer at prefill 512 with router bias b_e = 1.5 ln(1/(e+1)^1.1)
    C2  H 2048, E 512, top-10 softmax, F 512, IQ2_XS experts, one shared
        expert (F 512, Q8_0) gated by sigmoid(v . x); batch 1 and 4
    C3  GLM-style: H 4096, E 128, top-8 on sigmoid(l) + U(-0.1, 0.1) bias,
        weights normalised over the selected sigmoid scores (scale 1), F 1408,
        IQ3_XXS gate/up, IQ4_NL down (Q4_K cannot hold 1408 columns: GGUF
        needs a multiple of 256), ungated shared expert (F 1408), 64 tokens,
        x rounded to bf16
    C4  48 stacked C0-shaped layers with RMSNorm (eps 1e-6, gain N(1, 0.02))
        and a residual add: h <- h + MoE_l(RMSNorm_l(h)); batch 1 and 8
"""
from __future__ import annotations

import math
import os
from typing import Optional

import numpy as np

from . import _native as N
from .moe import (IQ2_XS, IQ3_XXS, IQ4_NL, Q4_K, Q8_0, ROUTE_SIGMOID, ROUTE_SOFTMAX, LayerSpec, Matrix)

# tensor ids in the stream key
T_ROUTER, T_GATE, T_UP, T_DOWN, T_SGATE, T_SUP, T_SDOWN, T_SGVEC, T_BIAS, T_GAIN, T_X = range(11)


def threads() -> int:
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(16, os.cpu_count() or 1))


def stream(config: int, layer: int, tensor: int, extra: int = 0) -> int:
    return int(N.synth_lib().ingot_synth_stream(config, layer, tensor, extra))


def normal(key: int, rows: int, cols: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    N.synth_lib().ingot_synth_normal(key, rows, cols, mean, sigma, out.ctypes.data, threads())
    return out


def uniform(key: int, rows: int, cols: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    N.synth_lib().ingot_synth_uniform(key, rows, cols, lo, hi, out.ctypes.data, threads())
    return out


def round_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32).copy()
    N.synth_lib().ingot_round_bf16(a.ctypes.data, a.size)
    return a


def row_bytes(kind: int, cols: int) -> int:
    n = int(N.synth_lib().ingot_quant_row_bytes(kind, cols))
    if n == 0:
        raise ValueError(f"kind {kind} cannot hold {cols} columns")
    return n


def quantize(kind: int, w: np.ndarray) -> Matrix:
    """w: [count, rows, cols] or [rows, cols] float32 -> Matrix."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.ndim == 2:
        w = w[None]
    count, rows, cols = w.shape
    stride = row_bytes(kind, cols)
    data = np.empty(count * rows * stride, np.uint8)
    if N.synth_lib().ingot_quantize(kind, w.ctypes.data, count * rows, cols, data.ctypes.data, threads()) != 0:
        raise ValueError("quantize failed")
    return Matrix(data, cols, rows, count, kind, stride)


def synth_matrix(kind: int, key: int, count: int, rows: int, cols: int, sigma: float = 0.02) -> Matrix:
    stride = row_bytes(kind, cols)
    data = np.empty(count * rows * stride, np.uint8)
    if N.synth_lib().ingot_synth_quantized(kind, key, count, rows, cols, sigma, data.ctypes.data, threads()) != 0:
        raise ValueError("synth_quantized failed")
    return Matrix(data, cols, rows, count, kind, stride)


def make_layer(config: int, layer: int, H: int, E: int, K: int, F: int, gate_kind: int, down_kind: int, *,
               routing: int = ROUTE_SOFTMAX, route_scale: float = 1.0, bias: Optional[str] = None,
               shared_ffn: int = 0, shared_gate_kind: Optional[int] = None, shared_down_kind: Optional[int] = None,
               shared_gated: bool = False, norm: bool = False, sigma: float = 0.02) -> LayerSpec:
    """A synthetic layer. bias: None, 'zipf' (b_e = 1.5 ln((e+1)^-1.1)) or 'uniform' (U(-0.1, 0.1))."""
    s = lambda t, e=0: stream(config, layer, t, e)  # noqa: E731
    router = normal(s(T_ROUTER), E, H, 0.0, sigma)
    gate = synth_matrix(gate_kind, s(T_GATE), E, F, H, sigma)
    up = synth_matrix(gate_kind, s(T_UP), E, F, H, sigma)
    down = synth_matrix(down_kind, s(T_DOWN), E, H, F, sigma)
    rb = None
    if bias == "zipf":
        rb = np.array([1.5 * math.log((e + 1.0) ** -1.1) for e in range(E)], np.float32)
    elif bias == "uniform":
        rb = uniform(s(T_BIAS), 1, E, -0.1, 0.1)[0]
    shared = None
    sgvec = None
    if shared_ffn:
        sk = shared_gate_kind if shared_gate_kind is not None else gate_kind
        dk = shared_down_kind if shared_down_kind is not None else down_kind
        shared = (synth_matrix(sk, s(T_SGATE), 1, shared_ffn, H, sigma),
                  synth_matrix(sk, s(T_SUP), 1, shared_ffn, H, sigma),
                  synth_matrix(dk, s(T_SDOWN), 1, H, shared_ffn, sigma))
        if shared_gated:
            sgvec = normal(s(T_SGVEC), 1, H, 0.0, sigma)[0]
    gain = normal(s(T_GAIN), 1, H, 1.0, 0.02)[0] if norm else None
    return LayerSpec(hidden=H, experts=E, top_k=K, router=router, gate=gate, up=up, down=down, routing=routing,
                     route_scale=route_scale, router_bias=rb, shared=shared, shared_gate_vec=sgvec, norm_gain=gain,
                     norm_eps=1e-6, meta={"config": config, "layer": layer})


def inputs(config: int, T: int, H: int, seed: int = 0, bf16: bool = False) -> np.ndarray:
    """x ~ N(0, 1) [T, H] from stream (config, seed, T_X)."""
    x = normal(stream(config, seed, T_X), T, H, 0.0, 1.0)
    return round_bf16(x) if bf16 else x


# ---- the BASELINE configurations ----
def c0_layer(layer: int = 0) -> LayerSpec:
    return make_layer(0, layer, 2048, 128, 8, 768, Q4_K, Q4_K)


def c1_layer() -> LayerSpec:
    spec = make_layer(0, 0, 2048, 128, 8, 768, Q4_K, Q4_K, bias="zipf")
    return spec


def c2_layer() -> LayerSpec:
    return make_layer(2, 0, 2048, 512, 10, 512, IQ2_XS, IQ2_XS, shared_ffn=512, shared_gate_kind=Q8_0,
                      shared_down_kind=Q8_0, shared_gated=True)


def c3_layer(route_scale: float = 1.0) -> LayerSpec:
    return make_layer(3, 0, 4096, 128, 8, 1408, IQ3_XXS, IQ4_NL, routing=ROUTE_SIGMOID, route_scale=route_scale,
                      bias="uniform", shared_ffn=1408)


def c4_layer(layer: int) -> LayerSpec:
    return make_layer(4, layer, 2048, 128, 8, 768, Q4_K, Q4_K, norm=True)


CONFIG_TOKENS = {0: (1,), 1: (512,), 2: (1, 4), 3: (64,), 4: (1, 8)}
