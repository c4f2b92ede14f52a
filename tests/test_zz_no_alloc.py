"""GPU test of the allocation-free forward (ingot_layer_forward_static).

It has no counterpart in the reference: it is the forward for callers that
cannot allocate device memory, with its workspace in the library's static
device array. Its outputs must equal ingot_layer_forward's (the same kernels on
the same inputs: bit for bit) on two static calls in a row, the second with a
smaller input, at decode and prefill sizes; a T whose workspace exceeds the
array is refused before anything runs.
"""
import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd.moe import InvalidData, MoeLayer

pytestmark = pytest.mark.gpu

STATIC_BYTES = 32 << 20


def run(layer, gpu, x, static):
    T, H, K = x.shape[0], layer.spec.hidden, layer.spec.top_k
    dx = gpu.to_device(x)
    out, ids, w = gpu.buffer(4 * T * H), gpu.buffer(4 * T * K), gpu.buffer(4 * T * K)
    out.upload(np.full(T * H, np.nan, np.float32))
    (layer.forward_static if static else layer.forward)(dx, T, out, ids, w)
    gpu.synchronize()
    gpu.check_device_flags()
    return (out.download(np.float32, T * H), ids.download(np.uint32, T * K), w.download(np.float32, T * K))


@pytest.mark.parametrize("name,Ts", [("c0", (8, 1)), ("c2", (4, 1)), ("c1", (128, 40))])
def test_static_forward_matches_forward(gpu, name, Ts):
    spec = {"c0": CF.c0_layer, "c2": CF.c2_layer, "c1": CF.c1_layer}[name]()
    layer = MoeLayer(gpu, spec)
    xs = [CF.inputs(30, T, spec.hidden, seed=T) for T in Ts]
    for x in xs:
        assert layer.static_bytes(x.shape[0]) <= STATIC_BYTES
    refs = [run(layer, gpu, x, static=False) for x in xs]
    got = [run(layer, gpu, x, static=True) for x in xs]  # two static calls in a row, the second smaller
    for T, r, g in zip(Ts, refs, got):
        assert np.array_equal(g[1], r[1]), f"{name} T={T}: ids"
        assert np.array_equal(g[2], r[2]), f"{name} T={T}: routing weights"
        assert np.array_equal(g[0], r[0]), f"{name} T={T}: outputs"
        print(f"{name} T={T}: static forward bit-equal to forward", flush=True)
    layer.destroy()


@pytest.mark.parametrize("name,T", [("c0", 8), ("c1", 128)])
def test_static_forward_first_on_a_fresh_layer_allocates_nothing(gpu, name, T):
    """A layer that has never reserved: the static forward makes no workspace
    and no tiled weight copies (device free memory and the layer's weight
    bytes unchanged), and equals a later forward() bit for bit."""
    spec = {"c0": CF.c0_layer, "c1": CF.c1_layer}[name]()
    warm = MoeLayer(gpu, spec)  # loads the code objects and runtime state the static path uses
    x = CF.inputs(32, T, spec.hidden, seed=T)
    run(warm, gpu, x, static=True)
    warm.destroy()
    layer = MoeLayer(gpu, spec)
    wb = layer.weight_bytes()
    dx = gpu.to_device(x)
    H, K = spec.hidden, spec.top_k
    out, ids, w = gpu.buffer(4 * T * H), gpu.buffer(4 * T * K), gpu.buffer(4 * T * K)
    gpu.synchronize()
    free0, _ = gpu.mem_info()
    layer.forward_static(dx, T, out, ids, w)
    gpu.synchronize()
    free1, _ = gpu.mem_info()
    gpu.check_device_flags()
    got = (out.download(np.float32, T * H), ids.download(np.uint32, T * K), w.download(np.float32, T * K))
    assert layer.weight_bytes() == wb, "the static forward made weight copies"
    assert free0 - free1 < layer.static_bytes(T) // 2, f"device free memory fell by {free0 - free1} bytes"
    ref = run(layer, gpu, x, static=False)
    for a, b, what in zip(got, ref, ("outputs", "ids", "routing weights")):
        assert np.array_equal(a, b), f"{name} T={T}: {what}"
    print(f"{name} T={T}: fresh static forward allocated nothing ({free0 - free1} bytes of free memory moved), "
          f"bit-equal to forward()", flush=True)
    layer.destroy()


def test_static_forward_refuses_oversized_batches(gpu):
    spec = CF.c1_layer()
    layer = MoeLayer(gpu, spec)
    T = 512
    assert layer.static_bytes(T) > STATIC_BYTES
    dx = gpu.to_device(CF.inputs(31, T, spec.hidden))
    out = gpu.buffer(4 * T * spec.hidden)
    with pytest.raises(InvalidData):
        layer.forward_static(dx, T, out)
    layer.destroy()
