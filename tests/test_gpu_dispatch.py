"""Bit-exact parity of the prefill dispatch's integer outputs (k_dispatch).

The layout (counts, first offsets), the stable pair order and its inverse are
the reference's expert_layout / expert_pairs contract (kernels/prefill.metal:
7-38), restated by oracle_dispatch (pinned against the reference's plan() in
tests/test_oracle.py). Index work must match exactly, not merely produce the
right layer outputs: a wrong but self-consistent permutation would pass every
end-to-end test. The GPU tile list holds the same {expert, first, n} tiles (64
pairs each, or 128 when an expert can take more than 64 pairs, the batch
averages at least 32 pairs per expert and both projections are Q4_K or Q5_K
on the f16 GEMM) in its own order: the shared
expert's tiles first, then every full tile, then the partial tiles by
decreasing n; its fourth word is the number of non-empty tiles.
"""
import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd.moe import GEMM_FP32, IQ4_NL, Q4_K, Q8_0, MoeLayer

pytestmark = pytest.mark.gpu


def f16_tile(T, K, E):
    """Tile size of the f16 GEMM's dispatch for Q4_K/Q5_K projections."""
    return 128 if T > 64 and T * K >= 32 * E else 64


def check_dispatch(layer, spec, x, oracle, label, tile=64):
    out, ids, _ = layer(x)
    T, K, E = x.shape[0], spec.top_k, spec.experts
    P = T * K
    d = layer.dispatch_debug(T)
    TILE = d["tile"]
    assert TILE == tile, f"{label}: {TILE}-pair tiles, expected {tile}"
    cap = P // TILE + E + 1
    used, counts, first, pairs, inverse, otiles = oracle.dispatch(ids.ravel(), E, TILE, cap)
    assert np.array_equal(d["counts"], counts), f"{label}: counts"
    assert np.array_equal(d["first"], first), f"{label}: first"
    assert np.array_equal(d["pairs"][:P], pairs), f"{label}: pairs"
    assert np.array_equal(d["inverse"], inverse), f"{label}: inverse"
    S = d["shared_rows"]
    tiles = d["tiles"]
    nt = int(tiles[0, 3]) if len(tiles) else 0
    assert (tiles[:, 3] == nt).all(), f"{label}: tile count word"
    live = tiles[:nt]
    assert not tiles[nt:, :3].any(), f"{label}: padding tiles"
    routed = live[live[:, 0] < E]
    shared = live[live[:, 0] == E]
    # the same routed tiles as the reference layout, as a set
    got = sorted(map(tuple, routed[:, :3].tolist()))
    ref = sorted(map(tuple, otiles[:used, :3].tolist()))
    assert got == ref, f"{label}: routed tiles"
    # order: shared tiles first, full tiles, then partial tiles by decreasing n
    ns = len(shared)
    assert (live[:ns, 0] == E).all()
    n_routed = live[ns:, 2]
    nfull = int((n_routed == TILE).sum())
    assert (n_routed[:nfull] == TILE).all(), f"{label}: full tiles first"
    assert (np.diff(n_routed[nfull:].astype(np.int64)) <= 0).all(), f"{label}: partial tiles by decreasing n"
    if S:
        assert S == T
        assert np.array_equal(d["pairs"][P:P + S], np.arange(T, dtype=np.uint32) * K), f"{label}: shared rows"
        exp = [(E, P + TILE * j, min(TILE, T - TILE * j)) for j in range((T + TILE - 1) // TILE)]
        assert list(map(tuple, shared[:, :3].tolist())) == exp, f"{label}: shared tiles"
    else:
        assert ns == 0
    print(f"{label}: {P} pairs, {len(routed)} routed tiles, {ns} shared tiles: dispatch bit-exact", flush=True)
    return ids


@pytest.mark.parametrize("T,seed", [(512, 0), (333, 1), (9, 2), (4096, 3)])
def test_dispatch_c1_zipf(gpu, oracle, T, seed):
    """C1's Zipf-biased routing: a hot expert with every token, empty experts."""
    spec = CF.c1_layer()
    layer = MoeLayer(gpu, spec)
    ids = check_dispatch(layer, spec, CF.inputs(1, T, 2048, seed=seed), oracle, f"C1 T={T}",
                         tile=f16_tile(T, spec.top_k, spec.experts))
    if T >= 512:
        counts = np.bincount(ids.ravel(), minlength=128)
        assert counts.max() == T and (counts == 0).any()
    layer.destroy()


def test_dispatch_tile_tails(gpu, oracle):
    """Expert loads around the tile size (1, 15, 16, 17, 31, 32, 33, 63, 64, 65,
    129, and a second 64 that brings the batch to 128-pair tiles) and empty
    experts, through an identity router."""
    E, K, H = 16, 1, 1024
    loads = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 129, 64, 0, 0, 0, 0]
    T = sum(loads)
    spec = CF.make_layer(11, E, H, E, K, 256, Q4_K, Q4_K)
    spec.router = np.zeros((E, H), np.float32)
    spec.router[np.arange(E), np.arange(E)] = 1.0
    x = CF.inputs(12, T, H) * 0.05
    order = np.repeat(np.arange(E), loads)
    np.random.default_rng(5).shuffle(order)
    x[:, :E] = 0.0
    x[np.arange(T), order] = 4.0
    layer = MoeLayer(gpu, spec)
    assert f16_tile(T, K, E) == 128
    check_dispatch(layer, spec, x, oracle, "tails", tile=128)
    layer.set_gemm_mode(GEMM_FP32)
    check_dispatch(layer, spec, x, oracle, "tails, fp32 GEMM", tile=64)
    layer.destroy()


def test_dispatch_many_experts(gpu, oracle):
    """1024 experts, top-16 (16 ids per token across every wave's histogram)."""
    spec = CF.make_layer(13, 0, 1024, 1024, 16, 64, Q8_0, Q8_0)
    layer = MoeLayer(gpu, spec)
    check_dispatch(layer, spec, CF.inputs(13, 40, 1024), oracle, "E=1024 K=16 T=40")
    layer.destroy()


def test_dispatch_with_merged_shared_expert(gpu, oracle):
    """A shared expert with the routed experts' formats and width runs in the
    same GEMM launches as expert id E over rows P..P+T-1."""
    spec = CF.make_layer(14, 0, 2048, 32, 4, 512, IQ4_NL, IQ4_NL, shared_ffn=512)
    layer = MoeLayer(gpu, spec)
    check_dispatch(layer, spec, CF.inputs(14, 150, 2048), oracle, "merged shared T=150")
    layer.destroy()
