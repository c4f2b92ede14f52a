"""ctypes wrapper of oracle/liboracle.so. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker or the timed CPU baseline.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# INGOT_ORACLE_LIB: another build of the same sources (the sanitizer build of
# `make -C oracle sanitize`).
LIB = os.environ.get("INGOT_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

OK, INVALID, NONFINITE = 0, 1, 2
F64, F32 = 64, 32


class OMatrix(C.Structure):
    _fields_ = [("data", C.c_void_p), ("nbytes", C.c_uint64), ("cols", C.c_uint64), ("rows", C.c_uint64),
                ("count", C.c_uint64), ("kind", C.c_uint32), ("stride", C.c_uint64)]


class OLayer(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("experts", C.c_uint32), ("top_k", C.c_uint32), ("routing", C.c_uint32),
                ("route_scale", C.c_float), ("swiglu_limit", C.c_float), ("router", C.c_void_p),
                ("router_bias", C.c_void_p), ("gate", OMatrix), ("up", OMatrix), ("down", OMatrix),
                ("has_shared", C.c_int), ("shared_gate", OMatrix), ("shared_up", OMatrix), ("shared_down", OMatrix),
                ("shared_gate_vec", C.c_void_p), ("norm_gain", C.c_void_p), ("norm_eps", C.c_float)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            subprocess.run(["make", "-s", "-C", HERE], check=True)
        L = C.CDLL(LIB)
        P, U32, U64, F = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float
        sig = {
            "oracle_geometry": (C.c_int, [U32, P, P]),
            "oracle_validate_matrix": (C.c_int, [C.POINTER(OMatrix)]),
            "oracle_dequant_value": (F, [P, U32, U64]),
            "oracle_dequant_row": (None, [P, U32, U64, P]),
            "oracle_route_softmax": (C.c_int, [P, U32, U32, P, P]),
            "oracle_route_sigmoid": (C.c_int, [P, P, U32, U32, F, P, P]),
            "oracle_router_logits": (None, [P, P, U32, U32, U32, P, C.c_int, P]),
            "oracle_project": (C.c_int, [C.POINTER(OMatrix), P, P]),
            "oracle_moe_forward": (C.c_int, [C.POINTER(OLayer), P, U32, P, P, P, C.c_int, C.c_int]),
            "oracle_dispatch": (U32, [P, U32, U32, U32, U32, P, P, P, P, P]),
            "oracle_det_expf": (F, [F]),
            "oracle_det_sigmoid": (F, [F]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def omatrix(m) -> OMatrix:
    d = np.ascontiguousarray(m.data, dtype=np.uint8)
    m.data = d
    return OMatrix(d.ctypes.data, d.nbytes, m.cols, m.rows, m.count, m.kind, m.stride)


def geometry(kind):
    b, n = C.c_uint32(), C.c_uint32()
    if lib().oracle_geometry(kind, C.byref(b), C.byref(n)) != OK:
        return None
    return b.value, n.value


def validate(m) -> bool:
    return lib().oracle_validate_matrix(C.byref(omatrix(m))) == OK


def dequant_rows(m) -> np.ndarray:
    """All count*rows rows of a Matrix as float32 [count*rows, cols]."""
    om = omatrix(m)
    out = np.empty((m.count * m.rows, m.cols), np.float32)
    base = m.data.ctypes.data
    for r in range(m.count * m.rows):
        lib().oracle_dequant_row(base + r * m.stride, m.kind, m.cols, out[r].ctypes.data)
    del om
    return out


def dequant_value(row_bytes: np.ndarray, kind: int, j: int) -> float:
    b = np.ascontiguousarray(row_bytes, dtype=np.uint8)
    return float(lib().oracle_dequant_value(b.ctypes.data, kind, j))


def route_softmax(logits, K):
    l = _f32(logits)
    ids = np.zeros(max(K, 1), np.uint32)
    w = np.zeros(max(K, 1), np.float32)
    st = lib().oracle_route_softmax(l.ctypes.data, l.size, K, ids.ctypes.data, w.ctypes.data)
    if st != OK:
        return None
    return ids[:K], w[:K]


def route_sigmoid(logits, bias, K, scale=1.0):
    l = _f32(logits)
    b = _f32(bias) if bias is not None else None
    ids = np.zeros(max(K, 1), np.uint32)
    w = np.zeros(max(K, 1), np.float32)
    st = lib().oracle_route_sigmoid(l.ctypes.data, b.ctypes.data if b is not None else None, l.size, K, scale,
                                    ids.ctypes.data, w.ctypes.data)
    if st != OK:
        return None
    return ids[:K], w[:K]


def router_logits(W, x, bias=None, add_bias=False):
    W, x = _f32(W), _f32(x)
    E, H = W.shape
    x = x.reshape(-1, H)
    T = x.shape[0]
    out = np.empty((T, E), np.float32)
    b = _f32(bias) if bias is not None else None
    lib().oracle_router_logits(W.ctypes.data, x.ctypes.data, T, E, H, b.ctypes.data if b is not None else None,
                               1 if add_bias else 0, out.ctypes.data)
    return out


def project(m, x) -> np.ndarray:
    x = _f32(x)
    y = np.empty(m.rows, np.float64)
    if lib().oracle_project(C.byref(omatrix(m)), x.ctypes.data, y.ctypes.data) != OK:
        raise ValueError("oracle_project: invalid matrix")
    return y


def _layer(spec, keep) -> OLayer:
    def ptr(a):
        if a is None:
            return None
        a = _f32(a)
        keep.append(a)
        return a.ctypes.data

    L = OLayer()
    L.hidden, L.experts, L.top_k, L.routing = spec.hidden, spec.experts, spec.top_k, spec.routing
    L.route_scale, L.swiglu_limit = spec.route_scale, spec.swiglu_limit
    L.router, L.router_bias = ptr(spec.router), ptr(spec.router_bias)
    L.gate, L.up, L.down = omatrix(spec.gate), omatrix(spec.up), omatrix(spec.down)
    if spec.shared is not None:
        L.has_shared = 1
        L.shared_gate, L.shared_up, L.shared_down = (omatrix(m) for m in spec.shared)
    L.shared_gate_vec, L.norm_gain = ptr(spec.shared_gate_vec), ptr(spec.norm_gain)
    L.norm_eps = spec.norm_eps
    return L


def moe_forward(spec, x, precision=F64, threads=0):
    """(status, out [T, H], ids [T, K], weights [T, K])."""
    keep = []
    L = _layer(spec, keep)
    x = _f32(x).reshape(-1, spec.hidden)
    T = x.shape[0]
    out = np.zeros((T, spec.hidden), np.float32)
    ids = np.zeros((T, spec.top_k), np.uint32)
    w = np.zeros((T, spec.top_k), np.float32)
    st = lib().oracle_moe_forward(C.byref(L), x.ctypes.data, T, out.ctypes.data, ids.ctypes.data, w.ctypes.data,
                                  precision, threads)
    return st, out, ids, w


def dispatch(ids, E, tile, cap):
    ids = np.ascontiguousarray(ids, dtype=np.uint32).ravel()
    P = ids.size
    counts = np.zeros(E, np.uint32)
    first = np.zeros(E, np.uint32)
    pairs = np.zeros(P, np.uint32)
    inverse = np.zeros(P, np.uint32)
    tiles = np.zeros((cap, 4), np.uint32)
    used = lib().oracle_dispatch(ids.ctypes.data, P, E, tile, cap, counts.ctypes.data, first.ctypes.data,
                                 pairs.ctypes.data, inverse.ctypes.data, tiles.ctypes.data)
    return int(used), counts, first, pairs, inverse, tiles


def det_expf(x: float) -> float:
    return float(lib().oracle_det_expf(x))


def det_sigmoid(x: float) -> float:
    return float(lib().oracle_det_sigmoid(x))
