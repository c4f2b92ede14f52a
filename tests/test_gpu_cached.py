"""Cached (bounded-memory) expert layers on the GPU: ingot_layer_create_cached,
the reference's ExpertWeights::Cached / ExpertCache (src/weights.rs:46-95) and
the cached branch of Qwen::ffn (src/qwen.rs:1171-1253). Routed experts stay in
host memory and are copied on demand into a few device slots; the forward runs
them in passes of at most `slots` experts.

Checks: oracle parity (ids exact, outputs to the bar) with fewer slots than the
experts a forward uses (several passes) and with one slot; outputs bit-equal to
the resident layer's on the same kernels; the hit / miss counters against the
cache policy driven with the forward's own routing (host-only
ingot_expert_cache_*, pinned per pass, experts in order of first use); shared
experts; graph capture refused."""
import ctypes as C

import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd.moe import IQ2_S, IQ2_XS, IQ3_S, IQ3_XXS, IQ4_NL, IQ4_XS, Q4_K, Q5_K, Q6_K, STAGE_DOWN, InvalidData, MoeLayer
from test_expert_cache import Cache
from util import check_layer

pytestmark = pytest.mark.gpu


def expected_stats(cache_slots, id_batches, bytes_per_expert):
    """Hits / misses / bytes of a sequence of forwards through the host-only
    policy: per forward, experts in order of first use, passes of at most
    `cache_slots` experts whose slots are pinned while the pass claims."""
    c = Cache(cache_slots)
    loads = 0
    for ids in id_batches:
        order = list(dict.fromkeys(int(e) for e in np.asarray(ids).ravel()))
        i = 0
        while i < len(order):
            pinned = []
            while i < len(order) and len(pinned) < cache_slots:
                before = c.state()[2]
                s = c.slot(order[i], pinned)
                assert s is not None
                loads += c.state()[2] - before
                pinned.append(s)
                i += 1
    _, hits, misses = c.state()
    c.close()
    return {"hits": hits, "misses": misses, "bytes": loads * bytes_per_expert}


@pytest.mark.parametrize("slots", [1, 3, 8])
def test_cached_layer_parity_and_counters(gpu, oracle, slots):
    spec = CF.make_layer(31, 0, 1024, 16, 4, 256, Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec, cache_slots=slots)
    batches = []
    for T, seed in ((1, 0), (3, 1), (40, 2), (1, 3)):
        out, ids, _ = check_layer(layer, spec, CF.inputs(31, T, 1024, seed=seed), oracle,
                                  f"cached slots={slots} T={T}")
        batches.append(ids)
    exp = expected_stats(slots, batches, spec.weight_bytes_per_expert())
    assert layer.cache_stats() == exp, (layer.cache_stats(), exp)
    layer.destroy()


@pytest.mark.parametrize("gk,dk", [(Q4_K, Q4_K), (Q5_K, Q5_K), (Q6_K, Q6_K), (Q4_K, Q6_K), (IQ2_XS, IQ2_XS),
                                   (IQ2_S, IQ4_XS), (IQ3_XXS, IQ4_NL), (IQ3_S, IQ3_S)])
def test_cached_equals_resident_bit_for_bit(gpu, gk, dk):
    """Prefill path, 160 pairs, merged shared expert. The resident layer's f16
    GEMMs read the tiled weight copies, the cached layer's read its slots in
    GGUF order; both decode the same operands and run the same products and
    combine, so the outputs are identical (which pins each tiled layout)."""
    spec = CF.make_layer(32, 0, 2048, 32, 4, 512, gk, dk, shared_ffn=512)
    x = CF.inputs(32, 40, 2048)
    res = MoeLayer(gpu, spec)
    cached = MoeLayer(gpu, spec, cache_slots=5)
    o1, i1, w1 = res(x)
    o2, i2, w2 = cached(x)
    assert res.stage_kernel(STAGE_DOWN) == "k_gemm_f16<down>"
    assert np.array_equal(i1, i2) and np.array_equal(w1, w2)
    assert np.array_equal(o1, o2)
    assert cached.cache_stats()["misses"] == len(np.unique(i2))
    res.destroy()
    cached.destroy()


def test_cached_shared_expert_unmerged(gpu, oracle):
    """A gated shared expert whose formats differ from the routed experts' (its
    own launches, run once in the first pass)."""
    spec = CF.make_layer(33, 0, 2048, 16, 4, 256, IQ4_NL, Q4_K, shared_ffn=512, shared_gate_kind=Q4_K,
                         shared_down_kind=IQ4_NL, shared_gated=True)
    layer = MoeLayer(gpu, spec, cache_slots=2)
    for T in (1, 24):
        check_layer(layer, spec, CF.inputs(33, T, 2048), oracle, f"cached unmerged shared T={T}")
    layer.destroy()


def test_cached_c2_shape(gpu, oracle):
    """configs[2]'s layer (512 IQ2_XS experts, top-10, gated Q8_0 shared expert)
    with 16 slots, at decode batch 1 and 4."""
    spec = CF.c2_layer()
    layer = MoeLayer(gpu, spec, cache_slots=16)
    batches = []
    for T in (1, 4):
        _, ids, _ = check_layer(layer, spec, CF.inputs(2, T, 2048), oracle, f"cached C2 b={T}")
        batches.append(ids)
    assert layer.cache_stats() == expected_stats(16, batches, spec.weight_bytes_per_expert())
    layer.destroy()


def test_cached_layer_refuses_capture_clone_and_static(gpu):
    spec = CF.make_layer(34, 0, 1024, 8, 2, 256, Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec, cache_slots=2)
    x = gpu.to_device(CF.inputs(34, 2, 1024))
    out = gpu.buffer(4 * 2 * 1024)
    layer.forward(x, 2, out)
    gpu.synchronize()
    with pytest.raises(InvalidData):
        layer.clone()
    with pytest.raises(InvalidData):
        layer.forward_static(x, 2, out)
    gpu.graph_begin()
    with pytest.raises(InvalidData):
        layer.forward(x, 2, out)
    try:
        gpu.graph_end().destroy()
    except Exception:
        pass
    layer.destroy()
    with pytest.raises(InvalidData):
        MoeLayer(gpu, spec, cache_slots=0)
    with pytest.raises(InvalidData):
        MoeLayer(gpu, spec, cache_slots=9)
