"""GPU parity tests of the MoE layer through the C ABI (libingot_moe.so).

Every test compares the HIP path with the CPU oracle (oracle/liboracle.so) on
the same seeded inputs: expert ids bit-exact, outputs within max-abs 1e-3 and
rel-L2 1e-4 (tests/util.py). Full BASELINE sizes run here too (C0, C1, C2,
C3, two stacked C4 layers).
"""
import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd.moe import (BF16, F16, IQ1_M, IQ2_S, IQ2_XS, IQ2_XXS, IQ3_S, IQ3_XXS, IQ4_NL, IQ4_XS, Q2_0, Q2_K, Q4_0,
                           Q4_K, Q5_K, Q6_K, Q8_0, ROUTE_SIGMOID, InvalidData, LayerSpec, Matrix,
                           MoeLayer, NonFinite)
from util import assert_close, check_layer

pytestmark = pytest.mark.gpu


def small_layer(gate_kind, down_kind, H=2048, E=16, K=4, F=256, **kw):
    return CF.make_layer(100 + gate_kind, down_kind, H, E, K, F, gate_kind, down_kind, **kw)


# ---------------------------------------------------------------- full configs
def test_c0_decode_full(gpu, oracle):
    spec = CF.c0_layer()
    layer = MoeLayer(gpu, spec)
    check_layer(layer, spec, CF.inputs(0, 1, 2048), oracle, "C0 decode b=1")
    layer.destroy()


def test_c1_prefill_full(gpu, oracle):
    spec = CF.c1_layer()
    layer = MoeLayer(gpu, spec)
    x = CF.inputs(1, 512, 2048)
    out, ids, _ = check_layer(layer, spec, x, oracle, "C1 prefill 512")
    counts = np.bincount(ids.ravel(), minlength=128)
    assert counts.max() > 100 and (counts == 0).any()  # Zipf-skewed load, empty experts
    layer.destroy()


def test_c1_prefill_4096_tokens(gpu, oracle):
    """Eight times the C1 batch: 32,768 pairs through one dispatch block, the
    hot expert (all but one token here) in 32 tiles of up to 128 pairs."""
    spec = CF.c1_layer()
    layer = MoeLayer(gpu, spec)
    x = CF.inputs(1, 4096, 2048, seed=5)
    out, ids, _ = check_layer(layer, spec, x, oracle, "C1 prefill 4096")
    assert np.bincount(ids.ravel(), minlength=128).max() > 31 * 128
    layer.destroy()


def test_c1_prefill_fp32_gemm_mode(gpu, oracle):
    """The fp32 MFMA GEMM (the path for non-Q4_K formats) on the C1 layer."""
    from ingot_amd.moe import GEMM_FP32
    spec = CF.c1_layer()
    layer = MoeLayer(gpu, spec)
    layer.set_gemm_mode(GEMM_FP32)
    check_layer(layer, spec, CF.inputs(1, 512, 2048, seed=1), oracle, "C1 prefill 512 fp32 GEMM")
    layer.destroy()


def test_c2_decode_full(gpu, oracle):
    spec = CF.c2_layer()
    layer = MoeLayer(gpu, spec)
    for T in (1, 4):
        check_layer(layer, spec, CF.inputs(2, T, 2048), oracle, f"C2 b={T}")
    layer.destroy()


def test_iq2s_iq3s_mix_decode_512_experts(gpu, oracle):
    """An IQ2_XS-class checkpoint's mix at configs[2]'s shape: IQ2_S gate/up and IQ3_S down
    over 512 experts (top-10), a gated shared expert with IQ4_XS gate/up and Q2_0 down of the
    routed width (it joins the routed decode kernels), at 1 and 4 tokens."""
    from ingot_amd.moe import IQ2_S, IQ3_S, IQ4_XS, Q2_0
    spec = CF.make_layer(2, 0, 2048, 512, 10, 512, IQ2_S, IQ3_S, shared_ffn=512, shared_gate_kind=IQ4_XS,
                         shared_down_kind=Q2_0, shared_gated=True)
    layer = MoeLayer(gpu, spec)
    for T in (1, 4):
        check_layer(layer, spec, CF.inputs(2, T, 2048, seed=T), oracle, f"IQ2_S/IQ3_S mix b={T}")
    layer.destroy()


def test_c3_prefill_full(gpu, oracle):
    spec = CF.c3_layer()
    layer = MoeLayer(gpu, spec)
    check_layer(layer, spec, CF.inputs(3, 64, 4096, bf16=True), oracle, "C3 T=64")
    layer.destroy()


def test_c4_48_stacked_layers_and_one_graph(gpu, oracle):
    """configs[4] at full depth: 48 independent C0-shaped layers with RMSNorm and
    the residual add, h <- h + MoE_l(RMSNorm_l(h)), at batch 1 and 8.
      * every layer against the oracle on the GPU's own input (ids exact,
        outputs to the bar);
      * the whole stack against the oracle's own 48-layer chain;
      * one HIP graph holding all 48 layers (the reference encodes one command
        buffer per decode token across layers, src/generic.rs:700-724),
        replayed three times with other work between, bit-equal to eager."""
    L = 48
    specs = [CF.c4_layer(l) for l in range(L)]
    layers = [MoeLayer(gpu, s) for s in specs]
    print("C4: 48 layers resident", flush=True)
    for T in (1, 8):
        h0 = CF.inputs(4, T, 2048)
        h, h_ref = h0, h0
        for l, (layer, spec) in enumerate(zip(layers, specs)):
            out, ids, w = layer(h)
            st, ref, rids, rw = oracle.moe_forward(spec, h, oracle.F64)
            assert st == 0 and np.array_equal(ids, rids), f"C4 layer {l} T={T}: ids"
            assert np.array_equal(w, rw), f"C4 layer {l} T={T}: routing weights"
            assert_close(out, ref, f"C4 layer {l} T={T}")
            st, h_ref, _, _ = oracle.moe_forward(spec, h_ref, oracle.F64)
            h = out
        m = assert_close(h, h_ref, f"C4 48-layer stack T={T}")
        print(f"C4 T={T}: 48 layers ids exact; stack vs oracle chain max-abs {m[0]:.2e} rel-L2 {m[1]:.2e}", flush=True)
        # eager on device buffers, then the same chain captured in one graph
        din = gpu.to_device(h0)
        bufs = [gpu.buffer(4 * T * 2048), gpu.buffer(4 * T * 2048)]

        def chain():
            src = din
            for l, layer in enumerate(layers):
                layer.forward(src, T, bufs[l & 1])
                src = bufs[l & 1]
            return bufs[(L - 1) & 1]
        res = chain()
        gpu.synchronize()
        gpu.check_device_flags()
        eager = res.download(np.float32, T * 2048).reshape(T, 2048)
        assert np.array_equal(eager, h), f"C4 T={T}: device chain differs from the per-layer calls"
        gpu.graph_begin()
        res = chain()
        g = gpu.graph_end()
        for rep in range(3):
            gpu.to_device(np.zeros(T * 2048, np.float32)).free()
            bufs[0].upload(np.full(T * 2048, 3.0, np.float32))
            bufs[1].upload(np.full(T * 2048, 5.0, np.float32))
            g.launch()
            gpu.synchronize()
            got = res.download(np.float32, T * 2048).reshape(T, 2048)
            assert np.array_equal(got, eager), f"C4 T={T}: graph replay {rep} differs from eager"
        g.destroy()
        print(f"C4 T={T}: one-graph 48-layer replays bit-equal to eager", flush=True)
    for layer in layers:
        layer.destroy()


# ------------------------------------------------------- formats and paths
@pytest.mark.parametrize("gk,dk", [(Q4_K, Q4_K), (Q8_0, Q8_0), (IQ4_NL, IQ4_NL), (IQ2_XS, IQ2_XS),
                                   (IQ3_XXS, IQ4_NL), (Q4_0, Q4_0), (Q4_K, Q8_0)])
def test_formats_decode_and_prefill(gpu, oracle, gk, dk):
    spec = small_layer(gk, dk)
    layer = MoeLayer(gpu, spec)
    for T in (1, 3, 40):  # 4 and 12 pairs: GEMV kernels; 160 pairs: grouped GEMM
        check_layer(layer, spec, CF.inputs(200 + gk, T, 2048), oracle, f"fmt {gk}/{dk} T={T}")
    layer.destroy()


NEW_FORMATS = [(Q2_K, Q2_K), (Q5_K, Q5_K), (Q6_K, Q6_K), (Q4_K, Q6_K), (IQ2_XXS, IQ2_XXS), (IQ2_S, IQ2_S),
               (IQ3_S, IQ3_S), (IQ4_XS, IQ4_XS), (IQ1_M, IQ1_M), (BF16, BF16), (F16, F16), (Q2_0, Q2_0),
               (IQ2_S, IQ4_XS), (IQ3_S, Q5_K), (IQ3_XXS, Q6_K)]


@pytest.mark.parametrize("gk,dk", NEW_FORMATS)
def test_remaining_formats_decode_and_prefill(gpu, oracle, gk, dk):
    """Every other type of the reference's table (kernels/moe.metal:17-89): decode
    GEMV kernels at 1 and 3 tokens, the fp32 grouped GEMM at 40 tokens."""
    spec = CF.make_layer(110, 100 * gk + dk, 1024, 16, 4, 256, gk, dk)
    layer = MoeLayer(gpu, spec)
    for T in (1, 3, 40):
        check_layer(layer, spec, CF.inputs(210 + gk, T, 1024), oracle, f"fmt {gk}/{dk} T={T}")
    layer.destroy()


@pytest.mark.parametrize("gemm_mode", ["auto", "fp32"])
def test_f16_gate_up_with_fp32_down(gpu, oracle, gemm_mode):
    """Q4_K gate/up on the f16 GEMM writing fp32 act for a down format without an
    f16 path (Q8_0) on the fp32 GEMM over the same tiles, with a shared expert
    beside them; the fp32 mode forces both onto the fp32 GEMM."""
    from ingot_amd.moe import GEMM_FP32
    spec = CF.make_layer(112, 0, 2048, 32, 8, 768, Q4_K, Q8_0, bias="zipf", shared_ffn=768,
                         shared_down_kind=Q8_0, shared_gated=True)
    layer = MoeLayer(gpu, spec)
    if gemm_mode == "fp32":
        layer.set_gemm_mode(GEMM_FP32)
    for T in (9, 200):
        check_layer(layer, spec, CF.inputs(212, T, 2048, seed=T), oracle, f"Q4_K/Q8_0 {gemm_mode} T={T}")
    if gemm_mode == "auto":
        from ingot_amd.moe import STAGE_DOWN, STAGE_GATEUP
        assert layer.stage_kernel(STAGE_GATEUP) == "k_gemm_f16<gate_up>"
        assert layer.stage_kernel(STAGE_DOWN) == "k_gemm<down>"
    layer.destroy()


@pytest.mark.parametrize("kind", [Q6_K, Q5_K, IQ1_M])
def test_remaining_formats_wide_hidden_many_experts_shared(gpu, oracle, kind):
    """H = 4096 (two chunks per lane), 256 experts (16 routing keys per lane),
    and a gated shared expert in the same format (separate GEMV pair)."""
    spec = CF.make_layer(111, kind, 4096, 256, 8, 256, kind, kind, shared_ffn=512, shared_gated=True)
    layer = MoeLayer(gpu, spec)
    for T in (1, 2, 24):
        check_layer(layer, spec, CF.inputs(211 + kind, T, 4096), oracle, f"fmt {kind} H=4096 E=256 T={T}")
    layer.destroy()


def test_forward_add_fuses_the_residual_add(gpu, oracle):
    """ingot_layer_forward_add(x, a): add_rms (kernels/generic.metal:390-405) fused
    into the router. Equals the oracle layer on s = x + a, and bit for bit the
    plain forward of x + a, at decode and prefill sizes; refused without a norm."""
    spec = CF.c4_layer(3)
    H, K = spec.hidden, spec.top_k
    layer = MoeLayer(gpu, spec)
    for T in (1, 8, 100):
        x = CF.inputs(40, T, H, seed=T)
        a = (0.5 * CF.inputs(41, T, H, seed=T)).astype(np.float32)
        s = (x + a).astype(np.float32)
        outs = []
        for fused in (True, False):
            o, i, w = gpu.buffer(4 * T * H), gpu.buffer(4 * T * K), gpu.buffer(4 * T * K)
            if fused:
                layer.forward_add(gpu.to_device(x), gpu.to_device(a), T, o, i, w)
            else:
                layer.forward(gpu.to_device(s), T, o, i, w)
            gpu.synchronize()
            outs.append((o.download(np.float32, T * H), i.download(np.uint32, T * K), w.download(np.float32, T * K)))
        assert all(np.array_equal(p, q) for p, q in zip(*outs)), f"T={T}: fused add differs from forward(x + a)"
        st, ref, rids, rw = oracle.moe_forward(spec, s, oracle.F64)
        assert st == 0 and np.array_equal(outs[0][1].reshape(T, K), rids)
        assert_close(outs[0][0].reshape(T, H), ref, f"forward_add T={T}")
    layer.destroy()
    plain = MoeLayer(gpu, small_layer(Q4_K, Q4_K, H=1024, E=8, K=2))
    with pytest.raises(InvalidData):
        plain.forward_add(gpu.to_device(np.zeros(1024, np.float32)), gpu.to_device(np.zeros(1024, np.float32)), 1,
                          gpu.buffer(4096))
    plain.destroy()


def test_hidden_4096_and_1024(gpu, oracle):
    for H in (4096, 1024, 2048):
        spec = small_layer(Q4_K, Q4_K, H=H, E=8, K=2, F=256)
        layer = MoeLayer(gpu, spec)
        for T in (1, 70):
            check_layer(layer, spec, CF.inputs(300 + H, T, H), oracle, f"H={H} T={T}")
        layer.destroy()


def test_shared_expert_gated_and_ungated(gpu, oracle):
    for gated, kinds in ((True, (IQ2_XS, Q8_0)), (False, (IQ3_XXS, IQ4_NL))):
        spec = CF.make_layer(7, int(gated), 2048, 32, 6, 512, kinds[0], kinds[0] if gated else kinds[1],
                             shared_ffn=512, shared_gate_kind=kinds[1] if gated else kinds[0],
                             shared_down_kind=kinds[1], shared_gated=gated)
        layer = MoeLayer(gpu, spec)
        for T in (1, 4, 33):
            check_layer(layer, spec, CF.inputs(7, T, 2048, seed=T), oracle, f"shared gated={gated} T={T}")
        layer.destroy()


BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ2_XS: 74, IQ2_S: 82, IQ3_XXS: 98, IQ3_S: 110, IQ4_NL: 18,
               IQ4_XS: 136}
D_OFFSET = {Q6_K: 208}  # byte offset of the block's f16 d (0 for the others)


def zero_scales(m, every=7, phase=3):
    """Sets d = 0 in every `every`-th block of a matrix (ggml writes such blocks for all-zero weights)."""
    bb, do = BLOCK_BYTES[m.kind], D_OFFSET.get(m.kind, 0)
    nblk = m.stride // bb
    blocks = m.data.copy().reshape(m.rows * m.count, nblk, bb)
    hit = (np.arange(blocks.shape[0] * nblk).reshape(-1, nblk) % every) == phase
    blocks[hit, do:do + 2] = 0
    m.data = blocks.reshape(-1)


def extreme_q6k_scales(m, seed):
    """Q6_K blocks with int8 scales drawn over all of [-128, 127] (|sc (q - 32)| up
    to 4096, odd products above 2048 included) and their d scaled down by 64."""
    rng = np.random.default_rng(seed)
    blocks = m.data.copy().reshape(-1, 210)
    blocks[:, 192:208] = rng.integers(0, 256, (blocks.shape[0], 16), dtype=np.uint8)
    d = blocks[:, 208:210].copy().view(np.float16) / np.float16(64)
    blocks[:, 208:210] = d.view(np.uint8)
    m.data = blocks.reshape(-1)


@pytest.mark.parametrize("gk,dk,sf", [(Q4_K, IQ4_NL, 512), (IQ3_XXS, Q4_K, 512), (IQ3_XXS, IQ3_XXS, 512),
                                      (IQ3_XXS, IQ4_NL, 256), (Q4_K, Q4_K, 512), (Q5_K, Q5_K, 512),
                                      (Q4_K, Q5_K, 512), (Q5_K, IQ4_NL, 256), (IQ2_XS, IQ2_XS, 512),
                                      (IQ2_XS, IQ4_NL, 512), (Q4_K, IQ2_XS, 256), (IQ4_NL, IQ4_NL, 512),
                                      (IQ4_NL, Q4_K, 256), (IQ4_XS, IQ4_XS, 512), (Q4_K, IQ4_XS, 512),
                                      (IQ4_XS, IQ2_XS, 256), (IQ2_S, IQ2_S, 512), (IQ2_S, IQ4_XS, 512),
                                      (Q4_K, IQ2_S, 256), (IQ3_S, IQ3_S, 512), (IQ2_S, IQ3_S, 256),
                                      (IQ3_S, IQ4_NL, 512), (Q6_K, Q6_K, 512), (Q4_K, Q6_K, 512),
                                      (Q6_K, IQ4_NL, 256), (IQ3_XXS, Q6_K, 256)])
def test_f16_gemm_formats_shared_and_zero_scales(gpu, oracle, gk, dk, sf):
    """Every format pair the f16 grouped GEMM takes, with a shared expert that joins its launches
    (same formats and width, sf == 512) or runs on the fp32 GEMM beside them (sf == 256), and
    blocks whose scale d is zero (unit 1, zeroed operand)."""
    spec = CF.make_layer(9, 10 * gk + dk, 2048, 16, 4, 512, gk, dk, shared_ffn=sf)
    for m in (spec.gate, spec.up, spec.down, *spec.shared):
        zero_scales(m)
    layer = MoeLayer(gpu, spec)
    from ingot_amd.moe import STAGE_DOWN, STAGE_GATEUP
    for T in (70, 130):  # 2 and 3 shared-expert tiles, partial last tiles
        check_layer(layer, spec, CF.inputs(9, T, 2048, seed=T), oracle, f"f16 {gk}/{dk} shared {sf} T={T}")
        # both projections ran on the f16 GEMM (not a silent fp32 fallback)
        assert layer.stage_kernel(STAGE_GATEUP) == "k_gemm_f16<gate_up>"
        assert layer.stage_kernel(STAGE_DOWN) == "k_gemm_f16<down>"
        assert not layer.last_fallback
    layer.destroy()


@pytest.mark.parametrize("extreme", [False, True])
def test_f16_q6k_down_unaligned_rows(gpu, oracle, extreme):
    """A Q4_K_M layer's shape (Qwen3-30B-A3B: F = 768, Q6_K down): 630-byte down
    rows, so every other row's superblocks start 2 bytes off a dword; a shared
    expert of the same formats in the same launches; blocks with d = 0; and
    (extreme) scales over the whole int8 range, so that B = sc (q - 32) needs
    its f16 remainder part."""
    from ingot_amd.moe import STAGE_DOWN, STAGE_GATEUP
    spec = CF.make_layer(113, int(extreme), 2048, 32, 8, 768, Q4_K, Q6_K, bias="zipf", shared_ffn=768,
                         shared_gated=True)
    for m in (spec.down, spec.shared[2]):
        if extreme:
            extreme_q6k_scales(m, seed=m.rows)
        zero_scales(m)
    layer = MoeLayer(gpu, spec)
    for T in (9, 70, 200):
        check_layer(layer, spec, CF.inputs(213, T, 2048, seed=T), oracle, f"Q4_K/Q6_K F=768 extreme={extreme} T={T}")
        if T > 8:
            assert layer.stage_kernel(STAGE_GATEUP) == "k_gemm_f16<gate_up>"
            assert layer.stage_kernel(STAGE_DOWN) == "k_gemm_f16<down>"
    layer.destroy()


def test_sigmoid_routing_scale_and_clamp(gpu, oracle):
    spec = small_layer(Q4_K, Q4_K, routing=ROUTE_SIGMOID, route_scale=2.5, bias="uniform")
    spec.swiglu_limit = 10.0
    layer = MoeLayer(gpu, spec)
    for T in (1, 50):
        check_layer(layer, spec, CF.inputs(8, T, 2048) * 3.0, oracle, f"sigmoid scale 2.5 clamp 10 T={T}")
    layer.destroy()


def test_decode_rows_independent_of_batch(gpu):
    """Batch-k decode rows equal batch-1 rows bitwise (src/expert_bench.rs:402-413)."""
    spec = small_layer(Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec)
    x = CF.inputs(9, 4, 2048)
    out4, ids4, w4 = layer(x)
    for t in range(4):
        out1, ids1, w1 = layer(x[t:t + 1])
        assert np.array_equal(out1[0], out4[t]) and np.array_equal(ids1[0], ids4[t])
    layer.destroy()


def test_decode_batches_c0_shape_odd_sizes(gpu, oracle):
    """configs[0]'s layer (128 experts, top-8, F = 768) at 2, 5 and 7 tokens on
    the decode kernels (three gate/up rows per wave, 256 row groups per
    token): the oracle's bar, and every row bit-equal to its one-token forward."""
    spec = CF.c0_layer()
    layer = MoeLayer(gpu, spec)
    for T in (2, 5, 7):
        x = CF.inputs(0, T, 2048, seed=T)
        out, ids, w = check_layer(layer, spec, x, oracle, f"C0 decode b={T}")
        for t in range(T):
            o1, i1, w1 = layer(x[t:t + 1])
            assert np.array_equal(o1[0], out[t]) and np.array_equal(i1[0], ids[t]) and np.array_equal(w1[0], w[t])
    layer.destroy()


# ---------------------------------------------------- dispatch edge cases
def identity_router_layer(E, K, H=1024, F=256, kind=Q4_K):
    """Router W = [I | 0]: logits[t] = x[t][:E] exactly, so x chooses the routing."""
    spec = CF.make_layer(11, E, H, E, K, F, kind, kind)
    spec.router = np.zeros((E, H), np.float32)
    spec.router[np.arange(E), np.arange(E)] = 1.0
    return spec


def test_dispatch_tile_tails_and_empty_experts(gpu, oracle):
    """Expert loads 1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 129 (tile tails at the 64-pair
    tile size and at the reference's 32) and empty experts, with ties in the logits."""
    E, K, H = 16, 1, 1024
    loads = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 129, 0, 0, 0, 0, 0]
    T = sum(loads)
    spec = identity_router_layer(E, K, H)
    x = CF.inputs(12, T, H) * 0.05
    order = np.repeat(np.arange(E), loads)
    rng = np.random.default_rng(5)
    rng.shuffle(order)
    x[:, :E] = 0.0
    x[np.arange(T), order] = 4.0
    x[:3, :E] = 1.0  # three tokens with all-tied logits: lowest id wins
    layer = MoeLayer(gpu, spec)
    out, ids, _ = check_layer(layer, spec, x, oracle, "dispatch tails")
    assert (ids[:3, 0] == 0).all()
    layer.destroy()


@pytest.mark.parametrize("kind", [Q4_K, Q5_K])
def test_f16_gemm_128_token_tiles(gpu, oracle, kind):
    """Batches in which an expert can take more than 64 pairs run the f16 GEMM on
    128-pair tiles: expert loads ending a tile at every 16-row block (1, 17, ...,
    113, 127), full tiles (128, 256) and tails past them (129, 200, 300), with a
    shared expert of the routed formats in the same launches."""
    from ingot_amd.moe import STAGE_DOWN, STAGE_GATEUP
    E, K, H, F = 16, 1, 1024, 512
    loads = [1, 17, 33, 49, 65, 81, 97, 113, 127, 128, 129, 200, 256, 300, 0, 0]
    T = sum(loads)
    spec = CF.make_layer(15, 0, H, E, K, F, kind, kind, shared_ffn=F)
    spec.router = np.zeros((E, H), np.float32)
    spec.router[np.arange(E), np.arange(E)] = 1.0
    x = CF.inputs(15, T, H) * 0.05
    order = np.repeat(np.arange(E), loads)
    np.random.default_rng(7).shuffle(order)
    x[:, :E] = 0.0
    x[np.arange(T), order] = 4.0
    layer = MoeLayer(gpu, spec)
    check_layer(layer, spec, x, oracle, f"128-token tiles kind {kind}")
    assert layer.stage_kernel(STAGE_GATEUP) == "k_gemm_f16<gate_up>"
    assert layer.stage_kernel(STAGE_DOWN) == "k_gemm_f16<down>"
    d = layer.dispatch_debug(T)
    assert d["tile"] == 128 and d["shared_rows"] == T
    want = sorted([128] * (l // 128) + [l % 128] * (l % 128 > 0) for l in loads + [T])
    want = sorted(v for w in want for v in w)
    got = sorted(int(v) for v in d["tiles"][:, 2] if v)
    assert got == want, "128-pair tiles: one per 128 pairs of an expert, then its tail"
    layer.destroy()


def test_route_ties_across_lanes_top8(gpu, oracle):
    E, K, H = 128, 8, 1024
    spec = identity_router_layer(E, K, H)
    x = CF.inputs(13, 6, H) * 0.05
    x[0, :E] = 1.0                                 # all tied
    x[1, :E] = ((np.arange(E) * 17) % 23) - 11.0   # many ties
    x[2, :E] = 0.0
    x[2, 70] = -0.0
    x[3, :E] = np.where(np.arange(E) % 64 == 5, 2.0, 0.0)  # ties at the same lane
    layer = MoeLayer(gpu, spec)
    out, ids, w = check_layer(layer, spec, x, oracle, "route ties")
    assert list(ids[0]) == list(range(8))
    layer.destroy()


@pytest.mark.parametrize("E,K", [(256, 10), (1024, 16)])
def test_decode_route_many_experts_ties(gpu, oracle, E, K):
    """Decode routing above 128 experts (each wave ranks its own keys; the waves' best K are then
    ranked against each other), with ties inside a wave, across waves and between the two keys a
    lane holds when E > 512: ids bit-exact, lower id first."""
    H = 1024
    spec = identity_router_layer(E, K, H, F=64, kind=Q8_0)
    x = CF.inputs(14, 4, H) * 0.05
    x[0, :E] = 1.0                                          # all tied: ids 0..K-1
    x[1, :E] = ((np.arange(E) * 17) % 23) - 11.0            # ties spread over every wave
    x[2, :E] = np.where(np.arange(E) % 64 == 9, 3.0, 0.0)   # ties at one lane of every wave
    x[3, :E] = np.where(np.arange(E) % 512 == 7, 2.0, 0.0)  # ties between a lane's two keys
    layer = MoeLayer(gpu, spec)
    out, ids, w = check_layer(layer, spec, x, oracle, f"route E={E} K={K}")
    assert list(ids[0]) == list(range(K))
    layer.destroy()


@pytest.mark.parametrize("E,K,kind", [(256, 8, Q8_0), (512, 10, IQ2_XS)])
def test_decode_route_one_token_ties(gpu, oracle, E, K, kind):
    """One-token decode above 128 experts, where every wave routes the token
    itself (wave_route) and, when each candidate has a wave, loads its
    candidate's rows before the ranks are formed (8-wave blocks at 256
    experts, 12-wave blocks for IQ2_XS at 512): all logits tied, a tie at the
    top among every 13th expert (20 or 40 candidates, more than the waves:
    the ranks come first), ties spread over the lanes, and untied logits.
    Ids bit-exact, lower id first."""
    H = 1024
    spec = identity_router_layer(E, K, H, F=256 if kind == IQ2_XS else 64, kind=kind)
    x = CF.inputs(15, 4, H) * 0.05
    x[0, :E] = 1.0
    x[1, :E] = np.where(np.arange(E) % 13 == 0, 2.0, 0.0)
    x[2, :E] = ((np.arange(E) * 17) % 23) - 11.0
    layer = MoeLayer(gpu, spec)
    for i in range(4):
        _, ids, _ = check_layer(layer, spec, x[i:i + 1], oracle, f"one-token route E={E} K={K} input {i}")
        if i == 0:
            assert list(ids[0]) == list(range(K))
        if i == 1:
            assert list(ids[0]) == [13 * j for j in range(K)]
    layer.destroy()


def test_tiled_copies_made_for_prefill_only(gpu, oracle):
    """The prefill GEMM's tiled weight copies appear at the first batch that
    takes the prefill path (never for decode), travel with clones, and leave
    the outputs as they were."""
    spec = small_layer(Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec)
    gguf = layer.weight_bytes()
    x1, x40 = CF.inputs(16, 1, 2048), CF.inputs(16, 40, 2048)
    out1, _, _ = check_layer(layer, spec, x1, oracle, "decode before any prefill")
    assert layer.weight_bytes() == gguf
    check_layer(layer, spec, x40, oracle, "first prefill")
    routed = sum(m.data.nbytes for m in (spec.gate, spec.up, spec.down))
    assert layer.weight_bytes() == gguf + routed
    assert np.array_equal(layer(x1)[0], out1)
    clone = layer.clone()
    assert clone.weight_bytes() == layer.weight_bytes()
    assert np.array_equal(clone(x40)[0], layer(x40)[0])
    clone.destroy()
    layer.destroy()


# ----------------------------------------------------------- errors, graphs
def test_nonfinite_input_rejected(gpu):
    spec = small_layer(Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec)
    x = CF.inputs(14, 2, 2048)
    x[1, 7] = np.nan
    with pytest.raises(NonFinite):
        layer(x)
    # device-side detection: the NaN reaches the router, the flag is raised
    d = gpu.to_device(x)
    out = gpu.buffer(4 * 2 * 2048)
    layer.forward(d, 2, out)
    with pytest.raises(NonFinite):
        gpu.check_device_flags()
    gpu.check_device_flags()  # cleared
    layer.destroy()


@pytest.mark.parametrize("case", ["decode", "decode_fused_shared", "decode_shared_add", "prefill"])
def test_nonfinite_output_flagged(gpu, oracle, case):
    """Finite inputs (N(0,1) x 1e25) whose expert products overflow fp32: the
    oracle rejects the output, and the kernel that writes the layer output
    (k_dec_down, k_gemv_shared_down_add, k_combine) raises the device flag;
    a finite forward afterwards raises nothing."""
    kw = {}
    if case == "decode_fused_shared":
        kw = dict(shared_ffn=256, shared_gate_kind=Q4_K, shared_down_kind=Q4_K)
    elif case == "decode_shared_add":
        kw = dict(shared_ffn=256, shared_gate_kind=Q8_0, shared_down_kind=Q8_0)
    spec = small_layer(Q4_K, Q4_K, **kw)
    T = 64 if case == "prefill" else 1
    x = CF.inputs(15, T, 2048) * np.float32(1e25)
    assert np.isfinite(x).all()
    assert oracle.moe_forward(spec, x, oracle.F64)[0] == oracle.NONFINITE
    layer = MoeLayer(gpu, spec)
    if case == "prefill":
        from ingot_amd.moe import GEMM_FP32
        layer.set_gemm_mode(GEMM_FP32)  # the split-f16 GEMM would report the range first
    d = gpu.to_device(x)
    out = gpu.buffer(4 * T * 2048)
    layer.forward(d, T, out)
    with pytest.raises(NonFinite, match="output"):
        gpu.check_device_flags()
    gpu.check_device_flags()  # cleared
    layer.forward(gpu.to_device(CF.inputs(15, T, 2048)), T, out)
    gpu.check_device_flags()
    with pytest.raises(NonFinite):
        layer(x)
    layer.destroy()


def test_layer_rejects_bad_shapes(gpu):
    spec = small_layer(Q4_K, Q4_K)
    bad = LayerSpec(**{**spec.__dict__})
    bad.down = Matrix(spec.down.data, spec.down.cols, spec.down.rows - 1, spec.down.count, spec.down.kind,
                      spec.down.stride)
    with pytest.raises(InvalidData):
        MoeLayer(gpu, bad)
    bad2 = LayerSpec(**{**spec.__dict__})
    bad2.top_k = spec.experts + 1
    with pytest.raises(InvalidData):
        MoeLayer(gpu, bad2)


@pytest.mark.parametrize("T", [1, 48])
def test_graph_replays_match_eager(gpu, T):
    spec = small_layer(Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec)
    x = CF.inputs(15, T, 2048)
    ref, _, _ = layer(x)
    dx = gpu.to_device(x)
    dout = gpu.buffer(4 * T * 2048)
    layer.reserve(T)
    gpu.graph_begin()
    layer.forward(dx, T, dout)
    g = gpu.graph_end()
    for _ in range(4):
        gpu.to_device(np.zeros(T * 2048, np.float32)).free()
        dout.upload(np.full(T * 2048, 7.0, np.float32))
        g.launch()
        gpu.synchronize()
        assert np.array_equal(dout.download(np.float32, T * 2048).reshape(T, 2048), ref)
    g.destroy()
    layer.destroy()


def test_clone_matches(gpu):
    spec = small_layer(Q4_K, Q4_K)
    layer = MoeLayer(gpu, spec)
    twin = layer.clone()
    x = CF.inputs(16, 5, 2048)
    a, _, _ = layer(x)
    b, _, _ = twin(x)
    assert np.array_equal(a, b)
    twin.destroy()
    layer.destroy()
