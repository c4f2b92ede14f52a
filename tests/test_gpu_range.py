"""GPU tests of the split-f16 operand range (include/ingot_moe.h,
ingot_layer_set_gemm_mode).

The f16-MFMA prefill GEMM and the v_dot2 decode formats split their operands
into f16 hi + lo after a per-token power-of-two scale. x may take any finite
values: at input scales 1e-4, 3e3 and 1e5 the layer must match the oracle
without falling back. The prefill activations are scaled from x's exponent;
weights far from the usual size put them outside the checked range, and the
forward must then report INGOT_RANGE (never a silent mismatch), after which the
host convenience recomputes on the fp32 GEMM.

The reference's fp32 kernels have no operand range limit
(kernels/qwen.metal:895-973; non-finite outputs rejected at
src/metal.rs:1575-1577), so the bar here is the same parity bar, made relative
to the output's scale for max-abs (the absolute 1e-3 assumes O(1) outputs).
"""
import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd.moe import (GEMM_FP32, IQ2_XS, Q4_K, STAGE_DOWN, STAGE_GATEUP, MoeLayer, OutOfRange)
from util import REL_L2, MAX_ABS, parity_metrics

pytestmark = pytest.mark.gpu


def assert_close_scaled(out, ref, what):
    maxabs, rel = parity_metrics(out, ref)
    scale = max(1.0, float(np.abs(np.asarray(ref, np.float64)).max()))
    assert maxabs <= MAX_ABS * scale and rel <= REL_L2, f"{what}: max-abs {maxabs:.3e} (scale {scale:.2e}) rel-L2 {rel:.3e}"
    return maxabs, rel


def check_scaled(layer, spec, x, oracle, label, fallback=False):
    out, ids, w = layer(x)
    st, o64, ids64, w64 = oracle.moe_forward(spec, x, oracle.F64)
    assert st == 0
    assert np.array_equal(ids, ids64), f"{label}: expert ids differ from the oracle"
    assert np.array_equal(w, w64), f"{label}: routing weights differ"
    m = assert_close_scaled(out, o64, label)
    assert layer.last_fallback == fallback, f"{label}: fallback {layer.last_fallback}, expected {fallback}"
    print(f"{label}: ids exact, max-abs {m[0]:.2e} rel-L2 {m[1]:.2e}, fallback {layer.last_fallback}", flush=True)
    return out


@pytest.fixture(scope="module")
def c1(gpu):
    spec = CF.c1_layer()
    layer = MoeLayer(gpu, spec)
    yield spec, layer
    layer.destroy()


@pytest.fixture(scope="module")
def c2(gpu):
    spec = CF.c2_layer()
    layer = MoeLayer(gpu, spec)
    yield spec, layer
    layer.destroy()


@pytest.mark.parametrize("scale", [1e-4, 3e3, 1e5])
def test_c1_shape_scaled_inputs(c1, oracle, scale):
    """Q4_K layer: decode (fp32 GEMVs) at 1 token, the f16 GEMM at 512 tokens."""
    spec, layer = c1
    for T in (1, 512):
        x = CF.inputs(1, T, 2048, seed=7) * np.float32(scale)
        check_scaled(layer, spec, x, oracle, f"C1 shape x*{scale:g} T={T}")
        if T == 512:
            assert layer.stage_kernel(STAGE_GATEUP) == "k_gemm_f16<gate_up>"
            assert layer.stage_kernel(STAGE_DOWN) == "k_gemm_f16<down>"


@pytest.mark.parametrize("scale", [1e-4, 3e3, 1e5])
def test_c2_shape_scaled_inputs(c2, oracle, scale):
    """IQ2_XS layer with a gated Q8_0 shared expert: the v_dot2 decode GEMVs
    (x and act split to f16 pairs) at 1 and 4 tokens, the f16 GEMM at 128."""
    spec, layer = c2
    for T in (1, 4, 128):
        x = CF.inputs(2, T, 2048, seed=7) * np.float32(scale)
        check_scaled(layer, spec, x, oracle, f"C2 shape x*{scale:g} T={T}")
    assert layer.stage_kernel(STAGE_GATEUP) == "k_gemm_f16<gate_up>"


def test_mixed_token_scales_one_batch(c1, oracle):
    """Tokens of very different magnitude in one prefill batch: each is split at
    its own scale."""
    spec, layer = c1
    x = CF.inputs(1, 256, 2048, seed=9)
    x *= np.logspace(-4, 5, 256, dtype=np.float64).astype(np.float32)[:, None]
    check_scaled(layer, spec, x, oracle, "C1 shape per-token scales 1e-4..1e5 T=256")


def test_zero_and_spiky_tokens(c1, oracle):
    """An all-zero token and tokens with a single large component."""
    spec, layer = c1
    x = CF.inputs(1, 96, 2048, seed=11)
    x[3] = 0.0
    x[5, 17] = 1e4
    x[40, 2000] = -3e3
    check_scaled(layer, spec, x, oracle, "C1 shape zero and spiky tokens T=96")


@pytest.mark.parametrize("sigma", [2.0, 2e-4])
def test_activations_out_of_range_report_and_fall_back(gpu, oracle, sigma):
    """Weights 100x larger or smaller than N(0, 0.02) put the prefill
    activations outside [2^-3, 2^14) of their scaled units: the forward raises
    the range flag (INGOT_RANGE), and the host convenience recomputes on the
    fp32 GEMM, matching the oracle."""
    spec = CF.make_layer(120, 0, 2048, 16, 4, 256, Q4_K, Q4_K, sigma=sigma)
    layer = MoeLayer(gpu, spec)
    T = 64
    x = CF.inputs(120, T, 2048)
    dx = gpu.to_device(x)
    dout = gpu.buffer(4 * T * 2048)
    layer.forward(dx, T, dout)
    with pytest.raises(OutOfRange):
        gpu.check_device_flags()
    gpu.check_device_flags()  # cleared
    check_scaled(layer, spec, x, oracle, f"Q4_K sigma {sigma} T={T}", fallback=True)
    # the fp32 GEMM itself raises nothing
    layer.set_gemm_mode(GEMM_FP32)
    layer.forward(dx, T, dout)
    gpu.check_device_flags()
    layer.destroy()


def test_in_range_layers_do_not_fall_back(gpu, oracle):
    """The usual weight scale keeps every f16 format's prefill on the f16 GEMM."""
    spec = CF.make_layer(121, 0, 2048, 16, 4, 512, IQ2_XS, Q4_K, sigma=0.02)
    layer = MoeLayer(gpu, spec)
    check_scaled(layer, spec, CF.inputs(121, 64, 2048), oracle, "IQ2_XS/Q4_K T=64")
    assert layer.stage_kernel(STAGE_GATEUP) == "k_gemm_f16<gate_up>"
    layer.destroy()
