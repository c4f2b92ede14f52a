"""GPU tests of the C ABI's lifetime rules and per-layer error attribution.

* Each layer raises its device flags in a word of its own, so a check after a
  stack of layers names the earliest-created flagged layer, and the engine
  recomputes from there (the reference fails the one command whose output is
  non-finite, src/metal.rs:1575-1577).
* A context with live layers cannot be destroyed (the reference gets the order
  from ownership: Gpu owns its buffers, src/metal.rs:46-63).
* Entry points that would replay or read a forward's buffers after they are
  gone refuse before launching anything: stage timing of a cached layer (its
  expert -> slot table exists only inside its forward), dispatch_debug after a
  static forward or after a reserve reallocated the workspace.
* The tiled weight copies are made only for matrices the f16 GEMM reads.
"""
import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd.moe import (GEMM_AUTO, GEMM_FP32, NONFINITE, OK, Q4_K, Q8_0, RANGE, STAGE_DOWN, STAGE_GATEUP, Gpu,
                           InvalidData, MoeLayer, NonFinite, OutOfRange)
from util import assert_close

pytestmark = pytest.mark.gpu


def chain(gpu, layers, x, T):
    """Runs the layers in sequence on device buffers and waits for them;
    returns every layer's output buffer."""
    src = gpu.to_device(x)
    outs = []
    for l in layers:
        dst = gpu.buffer(4 * T * l.spec.hidden)
        l.forward(src, T, dst)
        outs.append(dst)
        src = dst
    gpu.synchronize()
    return outs


def test_flagged_layer_is_named_and_suffix_recompute_matches_fp32(gpu, oracle):
    """Three prefill layers; only the middle one has weights 100x the usual
    size, which takes its split-f16 activations out of range. The check names
    layer 1 (creation order) and leaves layer 0 unflagged; recomputing layers
    1.. with layer 1 on the fp32 GEMM matches an all-fp32 run and the oracle."""
    T, H = 64, 2048
    specs = [CF.make_layer(130 + i, 0, H, 16, 4, 256, Q4_K, Q4_K, sigma=2.0 if i == 1 else 0.02) for i in range(3)]
    layers = [MoeLayer(gpu, s) for s in specs]
    x = CF.inputs(130, T, H)
    outs = chain(gpu, layers, x, T)
    with pytest.raises((OutOfRange, NonFinite)) as ei:
        gpu.check_device_flags()
    st = [l.flag_status() for l in layers]
    print("per-layer status:", st, "message:", ei.value, flush=True)
    assert st[0] == OK
    assert st[1] == RANGE
    assert isinstance(ei.value, OutOfRange), "the root cause (the first flagged layer) is reported"
    first = next(i for i, s in enumerate(st) if s != OK)
    assert first == 1 and "layer" in str(ei.value)
    gpu.check_device_flags()  # cleared
    assert [l.flag_status() for l in layers] == [OK, OK, OK]
    # suffix recompute from the first flagged layer: it on the fp32 GEMM, the rest as they were
    h0 = outs[0].download(np.float32, T * H).reshape(T, H)
    layers[1].set_gemm_mode(GEMM_FP32)
    suffix = chain(gpu, layers[1:], h0, T)
    gpu.check_device_flags()
    got = suffix[-1].download(np.float32, T * H).reshape(T, H)
    # all-fp32 run of the whole stack
    for l in layers:
        l.set_gemm_mode(GEMM_FP32)
    ref = chain(gpu, layers, x, T)[-1].download(np.float32, T * H).reshape(T, H)
    gpu.check_device_flags()
    scale = max(1.0, float(np.abs(ref).max()))
    assert_close(got / scale, ref / scale, "suffix recompute vs all-fp32 (scaled)")
    # and the oracle's chain
    h = x
    for s in specs:
        st_, h, _, _ = oracle.moe_forward(s, h, oracle.F64)
        assert st_ == 0
    assert_close(got / scale, h / scale, "suffix recompute vs the f64 oracle chain (scaled)")
    for l in layers:
        l.destroy()


def test_context_with_live_layer_cannot_be_destroyed(gpu):
    g2 = Gpu(0)
    layer = MoeLayer(g2, CF.make_layer(131, 0, 2048, 16, 4, 256, Q4_K, Q4_K))
    with pytest.raises(InvalidData, match="still alive"):
        g2.close()
    assert g2.ctx is not None
    x = CF.inputs(131, 1, 2048)
    layer(x)  # the context still works
    layer.destroy()
    g2.close()
    assert g2.ctx is None


def test_flag_words_are_per_layer_and_cleared_on_destroy(gpu):
    """A destroyed layer's unchecked flag does not leak into the next layer
    created in its slot."""
    bad = MoeLayer(gpu, CF.make_layer(132, 0, 2048, 16, 4, 256, Q4_K, Q4_K, sigma=2.0))
    T = 64
    dx = gpu.to_device(CF.inputs(132, T, 2048))
    dout = gpu.buffer(4 * T * 2048)
    bad.forward(dx, T, dout)
    gpu.synchronize()
    bad.destroy()  # flag raised, never checked
    good = MoeLayer(gpu, CF.make_layer(133, 0, 2048, 16, 4, 256, Q4_K, Q4_K))
    good.forward(dx, T, dout)
    gpu.check_device_flags()
    assert good.flag_status() == OK
    good.destroy()


def test_time_stage_refuses_cached_layers(gpu):
    spec = CF.make_layer(134, 0, 2048, 16, 4, 256, Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec, cache_slots=4)
    layer(CF.inputs(134, 32, 2048))
    for st in (STAGE_GATEUP, STAGE_DOWN):
        with pytest.raises(InvalidData, match="cached"):
            layer.time_stage(st, 4)
    layer.destroy()


def test_dispatch_debug_refused_after_static_forward_and_reallocation(gpu):
    spec = CF.make_layer(135, 0, 2048, 16, 4, 256, Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec)
    T = 32
    dx = gpu.to_device(CF.inputs(135, 2 * T, 2048))
    dout = gpu.buffer(4 * 2 * T * 2048)
    layer.forward(dx, T, dout)
    gpu.synchronize()
    assert layer.dispatch_debug(T)["counts"].sum() == T * 4
    layer.forward_static(dx, T, dout)
    with pytest.raises(InvalidData, match="static"):
        layer.dispatch_debug(T)
    layer.forward(dx, T, dout)
    layer.dispatch_debug(T)
    layer.reserve(2 * T)  # grows the workspace: the last forward's buffers are gone
    with pytest.raises(InvalidData):
        layer.dispatch_debug(T)
    with pytest.raises(InvalidData):
        layer.time_stage(STAGE_GATEUP, 4)
    gpu.check_device_flags()
    layer.destroy()


def test_tiled_copies_only_for_the_f16_gemm(gpu):
    """FP32 mode makes no tiled copies; AUTO makes them for the f16 GEMM's
    matrices only (a Q8_0 shared expert beside Q4_K routed experts is read by
    the fp32 GEMM and gets none)."""
    spec = CF.make_layer(136, 0, 2048, 16, 4, 256, Q4_K, Q4_K, shared_ffn=256, shared_gate_kind=Q8_0,
                         shared_down_kind=Q8_0)
    layer = MoeLayer(gpu, spec)
    base = layer.weight_bytes()
    layer.set_gemm_mode(GEMM_FP32)
    layer.reserve(64)
    assert layer.weight_bytes() == base
    layer.set_gemm_mode(GEMM_AUTO)
    layer.reserve(64)
    routed = sum(m.data.nbytes for m in (spec.gate, spec.up, spec.down))
    assert layer.weight_bytes() == base + routed
    layer.destroy()


def test_device_read_streams_and_captures(gpu):
    """ingot_device_read: eager and graph-captured, empty and non-empty."""
    n = 64 << 20
    buf = gpu.buffer(n)
    sink = gpu.buffer(4 * (n // 16384 + 2))
    gpu.stream_read(buf, n, sink)
    gpu.stream_read(buf, 0, sink)
    gpu.synchronize()
    gpu.graph_begin()
    gpu.stream_read(buf, n // 2, sink, offset=n // 2)
    gpu.stream_read(buf, 0, sink)
    g = gpu.graph_end()
    ms = g.time(3)
    g.destroy()
    assert ms > 0
    with pytest.raises(InvalidData):
        gpu._check(gpu.lib.ingot_device_read(gpu.ctx, buf.ptr, 17, sink.ptr))
    gpu.check_device_flags()
