"""Host-side mirror of Ingot's MoE-layer interface over the HIP backend.

Names, argument meaning and errors follow the reference:

* ``Matrix``      gguf::Matrix (src/gguf.rs:462-469) and ``geometry``
                  (src/gguf.rs:470-491)
* ``route``       route() (src/lib.rs:43-60): (ids, weights), raises
                  ``InvalidData`` for K == 0, K > E or non-finite logits
* ``Gpu``         Gpu::new / name / project / dequant / moe
                  (src/metal.rs:238, :1247, :1622, :1581, :1664)
* ``MoeLayer``    a resident MoE layer (all experts in HBM) and its forward,
                  the trunks' MoE FFN call (src/generic.rs:510-662,
                  src/qwen.rs:1062-1260, src/glm.rs:974-1060)

Every computation runs in libingot_moe.so on the GPU. There is no CPU
fallback: without the library or a GPU the calls raise.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _native as N

OK, INVALID, NONFINITE, DEVICE, UNSUPPORTED, RANGE = 0, 1, 2, 3, 4, 5
ROUTE_SOFTMAX, ROUTE_SIGMOID = 0, 1

# GGML type ids (src/gguf.rs:470-491)
F32, F16, Q4_0, Q8_0, Q4_K, IQ2_XS, IQ3_XXS, IQ4_NL = 0, 1, 2, 8, 12, 17, 18, 20
Q2_K, Q5_K, Q6_K, IQ2_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ1_M, BF16, Q2_0 = 10, 13, 14, 16, 21, 22, 23, 29, 30, 42

# Prefill GEMM arithmetic (ingot_layer_set_gemm_mode)
GEMM_AUTO, GEMM_FP32 = 0, 1

# Stages of a layer forward (ingot_layer_time_stage).
STAGE_ROUTER, STAGE_ROUTE, STAGE_GATEUP, STAGE_DOWN, STAGE_COMBINE, STAGE_DISPATCH = range(6)


class InvalidData(ValueError):
    """io::ErrorKind::InvalidData (src/lib.rs:39-41)."""


class NonFinite(InvalidData):
    """Non-finite input or output (src/metal.rs:1575-1577, :1680)."""


class Unsupported(InvalidData):
    """A GGML type or shape the kernels do not implement."""


class DeviceError(RuntimeError):
    """A HIP failure; the context refuses further work (src/metal.rs:1349-1353)."""


class OutOfRange(RuntimeError):
    """INGOT_RANGE: a prefill forward's activations left the range of the
    split-f16 GEMM; its outputs must be recomputed on the fp32 GEMM."""


def _raise(status: int, msg: str) -> None:
    if status == OK:
        return
    cls = {INVALID: InvalidData, NONFINITE: NonFinite, UNSUPPORTED: Unsupported,
           RANGE: OutOfRange}.get(status, DeviceError)
    raise cls(msg)


def geometry(kind: int) -> tuple[int, int]:
    """(values per block, bytes per block); InvalidData for unknown kinds."""
    lib = N.moe_lib()
    b, n = C.c_uint32(), C.c_uint32()
    if lib.ingot_geometry(kind, C.byref(b), C.byref(n)) != OK:
        raise InvalidData(f"GGML type {kind} is unsupported")
    return b.value, n.value


@dataclass
class Matrix:
    """gguf::Matrix: `count` matrices of rows x cols as GGUF block bytes."""

    data: np.ndarray  # uint8
    cols: int
    rows: int
    count: int
    kind: int
    stride: int

    def c(self) -> N.Matrix_t:
        d = np.ascontiguousarray(self.data, dtype=np.uint8)
        self.data = d
        return N.Matrix_t(d.ctypes.data, d.nbytes, self.cols, self.rows, self.count, self.kind, self.stride)

    def expert(self, e: int) -> "Matrix":
        n = self.rows * self.stride
        return Matrix(self.data[e * n:(e + 1) * n], self.cols, self.rows, 1, self.kind, self.stride)

    def select(self, ids: Sequence[int]) -> "Matrix":
        """The slabs of experts `ids`, in that order (what Gguf::matrix reads for
        ffn_weights, src/lib.rs:62-88, src/gguf.rs:434-460)."""
        n = self.rows * self.stride
        parts = [self.data[int(e) * n:(int(e) + 1) * n] for e in ids]
        return Matrix(np.concatenate(parts), self.cols, self.rows, len(parts), self.kind, self.stride)

    def validate(self) -> None:
        if N.moe_lib().ingot_validate_matrix(C.byref(self.c())) != OK:
            raise InvalidData("invalid quantized matrix layout")


def _empty_matrix() -> N.Matrix_t:
    return N.Matrix_t(None, 0, 0, 0, 0, 0, 0)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class DeviceBuffer:
    """Device memory owned through the library (no tensor framework needed)."""

    def __init__(self, gpu: "Gpu", nbytes: int):
        self.gpu = gpu
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        gpu._check(gpu.lib.ingot_malloc(gpu.ctx, self.nbytes, C.byref(p)))
        self.ptr = p.value

    def upload(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        self.gpu._check(self.gpu.lib.ingot_memcpy_h2d(self.gpu.ctx, self.ptr, a.ctypes.data, a.nbytes))
        return self

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        self.gpu._check(self.gpu.lib.ingot_memcpy_d2h(self.gpu.ctx, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def copy_from(self, src: "DeviceBuffer", nbytes: int) -> None:
        """Device-to-device copy by a plain HIP kernel (ingot_device_copy)."""
        assert nbytes <= min(self.nbytes, src.nbytes)
        self.gpu._check(self.gpu.lib.ingot_device_copy(self.gpu.ctx, self.ptr, src.ptr, int(nbytes)))

    def free(self) -> None:
        if self.ptr:
            self.gpu.lib.ingot_free(self.gpu.ctx, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Gpu:
    """Gpu::new(): one HIP device and stream; drop-in entry points of the reference's Gpu."""

    def __init__(self, device: int = 0):
        self.lib = N.moe_lib()
        ctx = C.c_void_p()
        st = self.lib.ingot_ctx_create(device, C.byref(ctx))
        if st != OK:
            _raise(st if st != INVALID else DEVICE, f"no usable HIP device {device}")
        self.ctx = ctx.value

    def close(self) -> None:
        """Destroys the context. Refused (InvalidData, the context kept) while
        layers created on it are alive: destroy them first."""
        if getattr(self, "ctx", None):
            st = self.lib.ingot_ctx_destroy(self.ctx)
            if st != OK:
                _raise(st, self.lib.ingot_last_error(self.ctx).decode())
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int) -> None:
        if st != OK:
            _raise(st, self.lib.ingot_last_error(self.ctx).decode())

    def name(self) -> str:
        return self.lib.ingot_device_name(self.ctx).decode()

    def synchronize(self) -> None:
        self._check(self.lib.ingot_ctx_synchronize(self.ctx))

    def check_device_flags(self) -> None:
        self._check(self.lib.ingot_ctx_check_device_flags(self.ctx))

    def stream_read(self, buf: DeviceBuffer, nbytes: int, sink: DeviceBuffer, offset: int = 0) -> None:
        """Asynchronous streaming read of nbytes at buf + offset by a plain
        kernel (ingot_device_read; nbytes == 0: an empty kernel node)."""
        assert offset + nbytes <= buf.nbytes and sink.nbytes >= 4 * max(1, -(-nbytes // 16384))
        self._check(self.lib.ingot_device_read(self.ctx, buf.ptr + offset, int(nbytes), sink.ptr))

    def mem_info(self) -> tuple[int, int]:
        """(free, total) bytes of device memory."""
        fr, to = C.c_uint64(), C.c_uint64()
        self._check(self.lib.ingot_device_mem_info(self.ctx, C.byref(fr), C.byref(to)))
        return fr.value, to.value

    def buffer(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        return DeviceBuffer(self, max(a.nbytes, 1)).upload(a)

    # -- route() --------------------------------------------------------
    def route(self, logits, top: int) -> tuple[list[int], np.ndarray]:
        l = _f32(logits)
        ids = np.zeros(max(top, 1), np.uint32)
        w = np.zeros(max(top, 1), np.float32)
        self._check(self.lib.ingot_route(self.ctx, l.ctypes.data, l.size, top, ids.ctypes.data, w.ctypes.data))
        return [int(i) for i in ids[:top]], w[:top]

    def route_batch(self, d_logits: DeviceBuffer, T: int, E: int, K: int, routing: int = ROUTE_SOFTMAX,
                    scale: float = 1.0, d_bias: Optional[DeviceBuffer] = None):
        ids = self.buffer(4 * T * K)
        w = self.buffer(4 * T * K)
        self._check(self.lib.ingot_route_batch(self.ctx, d_logits.ptr, d_bias.ptr if d_bias else None, T, E, K,
                                               routing, scale, ids.ptr, w.ptr))
        return ids, w

    # -- Gpu::project / dequant / moe ----------------------------------
    def project(self, m: Matrix, x) -> np.ndarray:
        x = _f32(x)
        if x.size != m.cols:
            raise InvalidData("projection shape mismatch")
        y = np.zeros(m.rows, np.float32)
        mt = m.c()
        self._check(self.lib.ingot_project(self.ctx, C.byref(mt), x.ctypes.data, y.ctypes.data))
        return y

    def dequant(self, m: Matrix) -> np.ndarray:
        out = np.zeros(m.cols * m.rows * m.count, np.float32)
        mt = m.c()
        self._check(self.lib.ingot_dequant(self.ctx, C.byref(mt), out.ctypes.data))
        return out

    def moe(self, routed: Sequence[Matrix], shared: Optional[Sequence[Matrix]], shared_gate: Optional[Matrix],
            x, weights) -> np.ndarray:
        x = _f32(x)
        w = _f32(weights)
        if routed[0].cols != x.size:
            raise InvalidData("MoE input shape mismatch")
        r = (N.Matrix_t * 3)(*[m.c() for m in routed])
        s = (N.Matrix_t * 3)(*[m.c() for m in shared]) if shared is not None else None
        g = C.byref(shared_gate.c()) if shared_gate is not None else None
        out = np.zeros(x.size, np.float32)
        self._check(self.lib.ingot_moe(self.ctx, r, s, g, x.ctypes.data, w.ctypes.data, w.size, out.ctypes.data))
        return out

    # -- graphs ----------------------------------------------------------
    def graph_begin(self) -> None:
        self._check(self.lib.ingot_graph_begin(self.ctx))

    def graph_end(self) -> "Graph":
        g = C.c_void_p()
        self._check(self.lib.ingot_graph_end(self.ctx, C.byref(g)))
        return Graph(self, g.value)


class Graph:
    def __init__(self, gpu: Gpu, handle):
        self.gpu, self.handle = gpu, handle

    def launch(self) -> None:
        self.gpu._check(self.gpu.lib.ingot_graph_launch(self.gpu.ctx, self.handle))

    def time(self, launches: int) -> float:
        ms = C.c_float()
        self.gpu._check(self.gpu.lib.ingot_graph_time(self.gpu.ctx, self.handle, launches, C.byref(ms)))
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            self.gpu.lib.ingot_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


@dataclass
class LayerSpec:
    """Host description of one MoE layer (ingot_layer_desc)."""

    hidden: int
    experts: int
    top_k: int
    router: np.ndarray  # [E, H] float32
    gate: Matrix
    up: Matrix
    down: Matrix
    routing: int = ROUTE_SOFTMAX
    route_scale: float = 1.0
    swiglu_limit: float = 0.0
    router_bias: Optional[np.ndarray] = None
    shared: Optional[tuple] = None  # (gate, up, down) Matrix
    shared_gate_vec: Optional[np.ndarray] = None
    norm_gain: Optional[np.ndarray] = None
    norm_eps: float = 1e-6
    meta: dict = field(default_factory=dict)

    @property
    def ffn(self) -> int:
        return self.gate.rows

    def weight_bytes_per_expert(self) -> int:
        return (self.gate.rows * self.gate.stride + self.up.rows * self.up.stride + self.down.rows * self.down.stride)

    def c(self) -> tuple[N.LayerDesc_t, list]:
        keep = []

        def ptr(a):
            if a is None:
                return None
            a = _f32(a)
            keep.append(a)
            return a.ctypes.data

        d = N.LayerDesc_t()
        d.hidden, d.experts, d.top_k, d.routing = self.hidden, self.experts, self.top_k, self.routing
        d.route_scale, d.swiglu_limit = self.route_scale, self.swiglu_limit
        d.router = ptr(self.router)
        d.router_bias = ptr(self.router_bias)
        d.gate, d.up, d.down = self.gate.c(), self.up.c(), self.down.c()
        if self.shared is not None:
            d.shared_gate, d.shared_up, d.shared_down = (m.c() for m in self.shared)
        else:
            d.shared_gate = d.shared_up = d.shared_down = _empty_matrix()
        d.shared_gate_vec = ptr(self.shared_gate_vec)
        d.norm_gain = ptr(self.norm_gain)
        d.norm_eps = self.norm_eps
        return d, keep


class MoeLayer:
    """A MoE layer on one GPU: every expert resident in HBM, or, with
    cache_slots, the routed experts kept in the spec's host bytes and copied on
    demand into that many device slots (ingot_layer_create_cached; the
    reference's ExpertWeights::Cached, src/weights.rs:46-95)."""

    def __init__(self, gpu: Gpu, spec: Optional[LayerSpec], _handle=None, cache_slots: Optional[int] = None):
        self.gpu = gpu
        self.spec = spec
        self.cache_slots = cache_slots
        if _handle is not None:
            self.handle = _handle
            return
        d, keep = spec.c()
        h = C.c_void_p()
        if cache_slots is None:
            gpu._check(gpu.lib.ingot_layer_create(gpu.ctx, C.byref(d), C.byref(h)))
        else:
            gpu._check(gpu.lib.ingot_layer_create_cached(gpu.ctx, C.byref(d), cache_slots, C.byref(h)))
            # the library reads the experts from these host bytes for the layer's lifetime
            self._host_experts = (keep, spec.gate.data, spec.up.data, spec.down.data)
        del keep
        self.handle = h.value

    def cache_stats(self) -> dict:
        """Cached layer: {"hits", "misses", "bytes"} since creation."""
        v = [C.c_uint64() for _ in range(3)]
        self.gpu._check(self.gpu.lib.ingot_layer_cache_stats(self.handle, *(C.byref(x) for x in v)))
        return {"hits": v[0].value, "misses": v[1].value, "bytes": v[2].value}

    def clone(self) -> "MoeLayer":
        h = C.c_void_p()
        self.gpu._check(self.gpu.lib.ingot_layer_clone(self.handle, C.byref(h)))
        return MoeLayer(self.gpu, self.spec, _handle=h.value)

    def destroy(self) -> None:
        if getattr(self, "handle", None):
            self.gpu.lib.ingot_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def weight_bytes(self) -> int:
        return int(self.gpu.lib.ingot_layer_weight_bytes(self.handle))

    def set_gemm_mode(self, mode: int) -> None:
        """GEMM_AUTO: split-precision f16 MFMA prefill for the formats that have it; GEMM_FP32: fp32 MFMA."""
        self.gpu._check(self.gpu.lib.ingot_layer_set_gemm_mode(self.handle, mode))
        self._gemm_mode = mode

    def reserve(self, T: int) -> None:
        self.gpu._check(self.gpu.lib.ingot_layer_reserve(self.handle, T))

    def forward(self, x: DeviceBuffer, T: int, out: DeviceBuffer, ids: Optional[DeviceBuffer] = None,
                weights: Optional[DeviceBuffer] = None) -> None:
        """Asynchronous on the context stream; device buffers in and out."""
        self.gpu._check(self.gpu.lib.ingot_layer_forward(self.handle, x.ptr, T, out.ptr, ids.ptr if ids else None,
                                                         weights.ptr if weights else None))

    def forward_static(self, x: DeviceBuffer, T: int, out: DeviceBuffer, ids: Optional[DeviceBuffer] = None,
                       weights: Optional[DeviceBuffer] = None) -> None:
        """forward() with the workspace in the library's static device array
        (ingot_layer_forward_static): allocates nothing; T is limited by
        static_bytes(T) <= 32 MiB; overlapping calls on one GPU race."""
        self.gpu._check(self.gpu.lib.ingot_layer_forward_static(self.handle, x.ptr, T, out.ptr,
                                                                ids.ptr if ids else None,
                                                                weights.ptr if weights else None))

    def static_bytes(self, T: int) -> int:
        return int(self.gpu.lib.ingot_layer_static_bytes(self.handle, T))

    def forward_add(self, x: DeviceBuffer, a: DeviceBuffer, T: int, out: DeviceBuffer,
                    ids: Optional[DeviceBuffer] = None, weights: Optional[DeviceBuffer] = None) -> None:
        """out = s + MoE(RMSNorm(s)), s = x + a (norm layers): add_rms fused into the router."""
        self.gpu._check(self.gpu.lib.ingot_layer_forward_add(self.handle, x.ptr, a.ptr, T, out.ptr,
                                                             ids.ptr if ids else None,
                                                             weights.ptr if weights else None))

    def __call__(self, x: np.ndarray):
        """Host convenience: out [T, H], ids [T, K], weights [T, K]. A forward
        that reports INGOT_RANGE (activations outside the split-f16 range) is
        recomputed on the fp32 GEMM; `last_fallback` tells whether it was."""
        x = _f32(x).reshape(-1, self.spec.hidden)
        T, H, K = x.shape[0], self.spec.hidden, self.spec.top_k
        if not np.isfinite(x).all():
            raise NonFinite("MoE input contains non-finite values")
        dx = self.gpu.to_device(x)
        dout = self.gpu.buffer(4 * T * H)
        dids = self.gpu.buffer(4 * T * K)
        dw = self.gpu.buffer(4 * T * K)
        self.forward(dx, T, dout, dids, dw)
        self.gpu.synchronize()
        self.last_fallback = False
        try:
            self.gpu.check_device_flags()
        except OutOfRange:
            mode = getattr(self, "_gemm_mode", GEMM_AUTO)
            self.set_gemm_mode(GEMM_FP32)
            try:
                self.forward(dx, T, dout, dids, dw)
                self.gpu.synchronize()
                self.gpu.check_device_flags()
            finally:
                self.set_gemm_mode(mode)
            self.last_fallback = True
        out = dout.download(np.float32, T * H).reshape(T, H)
        if not np.isfinite(out).all():
            raise NonFinite("output contains non-finite values")
        return out, dids.download(np.uint32, T * K).reshape(T, K), dw.download(np.float32, T * K).reshape(T, K)

    def flag_status(self) -> int:
        """What this layer's own forwards raised before the last
        Gpu.check_device_flags (OK, NONFINITE or RANGE)."""
        return int(self.gpu.lib.ingot_layer_flag_status(self.handle))

    def time_stage(self, stage: int, reps: int) -> float:
        ms = C.c_float()
        self.gpu._check(self.gpu.lib.ingot_layer_time_stage(self.handle, stage, reps, C.byref(ms)))
        return ms.value

    def stage_kernel(self, stage: int) -> str:
        return self.gpu.lib.ingot_layer_stage_kernel(self.handle, stage).decode()

    def dispatch_debug(self, T: int) -> dict:
        """The last prefill forward's dispatch arrays (ingot_layer_dispatch_debug)."""
        E, P = self.spec.experts, T * self.spec.top_k
        cap = P // 64 + E + T // 64 + 2
        counts, first = np.zeros(E, np.uint32), np.zeros(E, np.uint32)
        pairs, inverse = np.zeros(P + T, np.uint32), np.zeros(P, np.uint32)
        tiles = np.zeros((cap, 4), np.uint32)
        info = np.zeros(4, np.uint32)
        self.gpu._check(self.gpu.lib.ingot_layer_dispatch_debug(
            self.handle, counts.ctypes.data, first.ctypes.data, pairs.ctypes.data, inverse.ctypes.data,
            tiles.ctypes.data, cap, info.ctypes.data))
        P_, S, n, tile = (int(v) for v in info)
        assert P_ == P
        return {"counts": counts, "first": first, "pairs": pairs[:P + S], "inverse": inverse, "shared_rows": S,
                "tiles": tiles[:min(cap, n)], "tile": tile}


def time_stage(layers: Sequence[MoeLayer], stage: int, reps: int) -> float:
    """Mean ms per launch of one stage replayed round-robin over resident copies
    (graph-captured, HIP events on the context stream)."""
    gpu = layers[0].gpu
    arr = (C.c_void_p * len(layers))(*[l.handle for l in layers])
    ms = C.c_float()
    gpu._check(gpu.lib.ingot_layers_time_stage(arr, len(layers), stage, reps, C.byref(ms)))
    return ms.value


_default_gpu: Optional[Gpu] = None


def default_gpu() -> Gpu:
    global _default_gpu
    if _default_gpu is None:
        _default_gpu = Gpu(0)
    return _default_gpu


def route(logits, top: int) -> tuple[list[int], np.ndarray]:
    """route() (src/lib.rs:43-60) on the GPU: stable descending order by
    f32::total_cmp (ties to the lower id), top K, softmax over the selected."""
    l = _f32(logits)
    if top == 0 or top > l.size or not np.isfinite(l).all():
        raise InvalidData("invalid router scores or expert count")
    return default_gpu().route(l, top)
