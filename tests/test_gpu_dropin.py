"""GPU tests of the drop-ins for the reference's public API: route(), Gpu::project,
Gpu::dequant, Gpu::moe and device batch routing, against the reference's own
known answers (cited per test) and the CPU oracle."""
import math

import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd.moe import (BF16, F16, F32, IQ1_M, IQ2_S, IQ2_XS, IQ2_XXS, IQ3_S, IQ3_XXS, IQ4_NL, IQ4_XS, Q2_0, Q2_K,
                           Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, ROUTE_SIGMOID, ROUTE_SOFTMAX, InvalidData, Matrix)
from util import assert_close

pytestmark = pytest.mark.gpu


def test_route_reference_known_answer(gpu):
    """src/main.rs:340-349 (router_handles_large_logits_and_ties)."""
    ids, w = gpu.route([1000.0, -1000.0, 1000.0, 999.0], 3)
    assert ids == [0, 2, 3]
    assert abs(float(w.sum()) - 1.0) < 1e-6
    assert abs(w[0] / w[2] - math.e) < 1e-6
    for bad, k in (([math.nan], 1), ([0.0], 0), ([0.0], 2)):
        with pytest.raises(InvalidData):
            gpu.route(bad, k)


@pytest.mark.parametrize("E", [1, 31, 33, 63, 64, 65, 128, 288, 512, 1024])
@pytest.mark.parametrize("ties", [False, True])
def test_route_matches_oracle(gpu, oracle, E, ties):
    """src/metal/tests.rs:95-137 generator: logits ((i*17)%23)-11 or all 1000, K = min(E, 10)."""
    logits = np.full(E, 1000.0, np.float32) if ties else ((np.arange(E) * 17) % 23 - 11.0).astype(np.float32)
    K = min(E, 10)
    ids, w = gpu.route(logits, K)
    rids, rw = oracle.route_softmax(logits, K)
    assert ids == list(rids)
    assert np.array_equal(w, rw)
    # against route() in f64 (the reference test's 2e-5 bound on the weights)
    order = sorted(range(E), key=lambda i: -float(logits[i]))[:K]
    assert ids == order
    ex = np.exp(logits[order].astype(np.float64) - logits[order[0]])
    assert np.abs(w - ex / ex.sum()).max() < 2e-5


def test_route_signed_zero_total_order(gpu):
    """f32::total_cmp ranks +0.0 above -0.0 (src/lib.rs:48)."""
    ids, _ = gpu.route([-0.0, 0.0, -0.0, -1.0], 2)
    assert ids == [1, 0]


def test_route_batch_sigmoid_known_answer(gpu):
    """src/metal/tests.rs:306-322: logits [2,-2,0,2], bias [0,1,0,0], K=2, scale 2.5 -> ids [1,0]."""
    dl = gpu.to_device(np.array([2.0, -2.0, 0.0, 2.0], np.float32))
    db = gpu.to_device(np.array([0.0, 1.0, 0.0, 0.0], np.float32))
    ids, w = gpu.route_batch(dl, 1, 4, 2, ROUTE_SIGMOID, 2.5, db)
    gpu.synchronize()
    assert list(ids.download(np.uint32, 2)) == [1, 0]
    got = w.download(np.float32, 2)
    exp = [2.5 / (1.0 + math.exp(2.0)), 2.5 / (1.0 + math.exp(-2.0))]
    assert np.abs(got - exp).max() < 3e-5


@pytest.mark.parametrize("E", [1, 33, 288])
@pytest.mark.parametrize("ties", [False, True])
def test_route_batch_sigmoid_generator(gpu, oracle, E, ties):
    """src/metal/tests.rs:323-381 generator, several tokens per launch."""
    T = 3
    logits = np.zeros((T, E), np.float32) if ties else np.tile(((np.arange(E) % 7) - 3.0).astype(np.float32), (T, 1))
    bias = np.zeros(E, np.float32) if ties else (((np.arange(E) * 11) % 13) * 0.125).astype(np.float32)
    K = min(E, 8)
    ids, w = gpu.route_batch(gpu.to_device(logits), T, E, K, ROUTE_SIGMOID, 2.5, gpu.to_device(bias))
    gpu.synchronize()
    ids = ids.download(np.uint32, T * K).reshape(T, K)
    w = w.download(np.float32, T * K).reshape(T, K)
    for t in range(T):
        rids, rw = oracle.route_sigmoid(logits[t], bias, K, 2.5)
        assert np.array_equal(ids[t], rids) and np.array_equal(w[t], rw)
        score = 1.0 / (1.0 + np.exp(-logits[t].astype(np.float64))) + bias
        order = sorted(range(E), key=lambda i: -score[i])[:K]
        assert list(ids[t]) == order


def test_route_batch_softmax_bias(gpu, oracle):
    T, E, K = 7, 128, 8
    logits = CF.inputs(20, T, E) * 0.9
    bias = np.array([1.5 * math.log((e + 1.0) ** -1.1) for e in range(E)], np.float32)
    ids, w = gpu.route_batch(gpu.to_device(logits), T, E, K, ROUTE_SOFTMAX, 1.0, gpu.to_device(bias))
    gpu.synchronize()
    ids = ids.download(np.uint32, T * K).reshape(T, K)
    w = w.download(np.float32, T * K).reshape(T, K)
    for t in range(T):
        rids, rw = oracle.route_softmax((logits[t] + bias).astype(np.float32), K)
        assert np.array_equal(ids[t], rids) and np.array_equal(w[t], rw)


def test_project_f32_closed_form(gpu):
    """Closed form in the spirit of src/metal/tests.rs:14-33: weight row r is all (r+1),
    input all (j/32+1) -> y_r = (r+1) * sum_j (j/32+1)."""
    for rows in (1, 3, 4, 5, 7, 33):
        cols = 64
        w = np.repeat(np.arange(1, rows + 1, dtype=np.float32)[:, None], cols, 1)
        m = Matrix(w.view(np.uint8).ravel(), cols, rows, 1, F32, 4 * cols)
        x = (np.arange(cols) // 32 + 1).astype(np.float32)
        y = gpu.project(m, x)
        assert np.array_equal(y, (np.arange(1, rows + 1) * x.sum()).astype(np.float32))


def q4_0_fixture(rows, cols):
    """src/metal/tests.rs:42-52: Q4_0 blocks with fp16 scale 0.5 (0x3800) and nibbles
    low = (row + block + j) % 16, high = (row + block + j + 3) % 16."""
    data = bytearray()
    for row in range(rows):
        for block in range(cols // 32):
            data += (0x3800).to_bytes(2, "little")
            for j in range(16):
                data.append((((row + block + j + 3) % 16) << 4) | ((row + block + j) % 16))
    return np.frombuffer(bytes(data), np.uint8).copy()


def q4_0_expected(rows, cols):
    r = np.arange(rows)[:, None]
    j = np.arange(cols)[None, :]
    nib = (r + j // 32 + j % 16 + np.where(j % 32 >= 16, 3, 0)) % 16
    return (nib - 8.0) * 0.5


def test_q4_0_fixture_dequant_and_project(gpu):
    rows, cols = 35, 64
    m = Matrix(q4_0_fixture(rows, cols), cols, rows, 1, Q4_0, 36)
    assert np.array_equal(gpu.dequant(m).reshape(rows, cols), q4_0_expected(rows, cols).astype(np.float32))
    x = ((np.arange(cols) % 19) * 0.125 - 1.0).astype(np.float32)
    y = gpu.project(m, x)
    assert np.abs(y - q4_0_expected(rows, cols) @ x.astype(np.float64)).max() < 2e-5


@pytest.mark.parametrize("kind", [F32, Q4_0, Q8_0, Q4_K, IQ2_XS, IQ3_XXS, IQ4_NL])
def test_dequant_and_project_match_oracle(gpu, oracle, kind):
    cols = 512 if kind not in (Q4_K, IQ2_XS, IQ3_XXS) else 768
    w = CF.normal(CF.stream(30, kind, 0), 65, cols, 0.0, 0.02)
    m = CF.quantize(kind, w)
    got = gpu.dequant(m).reshape(65, cols)
    ref = oracle.dequant_rows(m)
    assert np.abs(got - ref).max() <= 1e-6 * max(1.0, np.abs(ref).max())
    x = CF.inputs(31, 1, cols)[0]
    y = gpu.project(m, x)
    yr = oracle.project(m, x)
    assert np.abs(y - yr).max() <= 1e-4 + 5e-5 * np.abs(yr).max()


@pytest.mark.parametrize("kind", [F16, BF16, Q2_K, Q5_K, Q6_K, IQ2_XXS, IQ2_S, IQ3_S, IQ4_XS, IQ1_M, Q2_0])
def test_dequant_and_project_remaining_formats(gpu, oracle, kind):
    """Gpu::dequant / Gpu::project (src/metal.rs:1581, :1622) on random valid blocks."""
    cols = 768
    m = CF.synth_matrix(kind, 32, 1, 65, cols)
    got = gpu.dequant(m).reshape(65, cols)
    ref = oracle.dequant_rows(m)
    assert np.abs(got - ref).max() <= 1e-6 * max(1.0, np.abs(ref).max())
    x = CF.inputs(33, 1, cols)[0]
    y = gpu.project(m, x)
    yr = oracle.project(m, x)
    assert np.abs(y - yr).max() <= 1e-4 + 5e-5 * np.abs(yr).max()


def test_moe_dropin_matches_oracle(gpu, oracle):
    """Gpu::moe (src/metal.rs:1664-1713) with K selected experts, a shared expert and its
    sigmoid gate, against the oracle layer routed to the same experts."""
    spec = CF.make_layer(40, 0, 2048, 8, 8, 256, Q4_K, Q4_K, shared_ffn=256, shared_gated=True)
    x = CF.inputs(40, 1, 2048)
    st, ref, ids, w = oracle.moe_forward(spec, x, oracle.F64)
    assert st == 0
    sel = list(ids[0])
    routed = [spec.gate.select(sel), spec.up.select(sel), spec.down.select(sel)]
    gvec = spec.shared_gate_vec.astype(np.float32)
    sgate = Matrix(gvec.view(np.uint8).copy(), 2048, 1, 1, F32, 4 * 2048)
    out = gpu.moe(routed, list(spec.shared), sgate, x[0], w[0])
    assert_close(out, ref[0], "Gpu::moe")


def test_moe_dropin_errors(gpu):
    spec = CF.make_layer(41, 0, 2048, 4, 2, 256, Q4_K, Q4_K)
    routed = [spec.gate.select([0, 1]), spec.up.select([0, 1]), spec.down.select([0, 1])]
    x = CF.inputs(41, 1, 2048)[0]
    with pytest.raises(InvalidData):
        gpu.moe(routed, None, None, x, np.array([0.5], np.float32))  # weights.len() != count
    xb = x.copy()
    xb[3] = np.inf
    with pytest.raises(InvalidData):
        gpu.moe(routed, None, None, xb, np.array([0.5, 0.5], np.float32))
    bad = Matrix(routed[2].data, routed[2].cols, routed[2].rows, routed[2].count, routed[2].kind, routed[2].stride + 1)
    with pytest.raises(InvalidData):
        gpu.moe([routed[0], routed[1], bad], None, None, x, np.array([0.5, 0.5], np.float32))
