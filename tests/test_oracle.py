"""CPU tests that pin the oracle (oracle/liboracle.so) before it is trusted.

Each check is independent of the oracle's own code path: the reference's known
answers (tests/golden/reference_known_answers.json), its dispatch generator
restated, exact rational arithmetic for the fixed reduction order, structural
(single-field) probes of every block layout, codebook checksums against the
reference's table text, and brute-force / closed-form layer math on small
shapes. No GPU.
"""
import hashlib
import json
import math
import os
import struct
from fractions import Fraction

import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd.moe import F32, IQ2_XS, IQ3_XXS, IQ4_NL, Q4_0, Q4_K, Q8_0, LayerSpec, Matrix

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "reference_known_answers.json")))
REFERENCE = "/root/reference"


def f16(x):
    return int(np.float16(x).view(np.uint16))


# ------------------------------------------------------------------ routing
def test_route_known_answer(oracle):
    g = GOLD["route_large_logits_and_ties"]
    ids, w = oracle.route_softmax(g["logits"], g["top"])
    assert list(ids) == g["ids"]
    assert abs(float(w.sum()) - g["sum"]) < 1e-6
    assert abs(w[0] / w[2] - g["w0_over_w2"]) < 1e-6
    for e in g["errors"]:
        l = [float(v) for v in e["logits"]]
        assert oracle.route_softmax(l, e["top"]) is None


@pytest.mark.parametrize("E", GOLD["routing_generators"]["softmax_counts"] + [63, 64, 65, 128])
@pytest.mark.parametrize("ties", [False, True])
def test_route_generator_matches_total_cmp_sort(oracle, E, ties):
    logits = np.full(E, 1000.0, np.float32) if ties else ((np.arange(E) * 17) % 23 - 11.0).astype(np.float32)
    K = min(E, 10)
    ids, w = oracle.route_softmax(logits, K)
    order = sorted(range(E), key=lambda i: -float(logits[i]))[:K]  # stable: ties keep the lower id
    assert list(ids) == order
    ex = np.exp(logits[order].astype(np.float64) - float(logits[order[0]]))
    assert np.abs(w - ex / ex.sum()).max() < 2e-5


def test_route_signed_zero_and_inf(oracle):
    ids, _ = oracle.route_softmax([-0.0, 0.0, -0.0, -1.0], 2)
    assert list(ids) == [1, 0]
    assert oracle.route_softmax([0.0, float("inf")], 1) is None


def test_glm_route_known_answer(oracle):
    g = GOLD["glm_route_bias_selects_scale_weights"]
    ids, w = oracle.route_sigmoid(g["logits"], g["bias"], g["top"], g["scale"])
    assert list(ids) == g["ids"]
    assert np.abs(w - np.array(g["weights"])).max() < 3e-5


@pytest.mark.parametrize("E", GOLD["routing_generators"]["sigmoid_counts"])
@pytest.mark.parametrize("ties", [False, True])
def test_glm_route_generator(oracle, E, ties):
    logits = np.zeros(E, np.float32) if ties else ((np.arange(E) % 7) - 3.0).astype(np.float32)
    bias = np.zeros(E, np.float32) if ties else (((np.arange(E) * 11) % 13) * 0.125).astype(np.float32)
    K = min(E, 8)
    ids, w = oracle.route_sigmoid(logits, bias, K, 2.5)
    score = 1.0 / (1.0 + np.exp(-logits.astype(np.float64))) + bias
    order = sorted(range(E), key=lambda i: -score[i])[:K]
    assert list(ids) == order
    sel = 1.0 / (1.0 + np.exp(-logits[order].astype(np.float64)))
    assert np.abs(w - sel / sel.sum() * 2.5).max() < 3e-5


def test_det_expf_and_sigmoid_accuracy(oracle):
    xs = np.concatenate([np.linspace(-103, 88.7, 4001), np.linspace(-1, 1, 2001), [0.0, -0.0, 1e-30, -1e-30]])
    for x in xs.astype(np.float32):
        got = oracle.det_expf(float(x))
        ref = math.exp(float(x))
        if ref < 1.2e-38:
            assert abs(got - ref) <= 2e-45 * 8
        else:
            assert abs(got - ref) <= 4 * np.spacing(np.float32(ref)), (x, got, ref)
    assert oracle.det_expf(89.0) == float("inf") and oracle.det_expf(-104.0) == 0.0
    for x in np.linspace(-30, 30, 601).astype(np.float32):
        assert abs(oracle.det_sigmoid(float(x)) - 1 / (1 + math.exp(-float(x)))) < 2e-7


# ------------------------------------------------------------- reduction order
def f32_round(v: Fraction) -> float:
    """Exact round-to-nearest-even of a rational to binary32."""
    if v == 0:
        return 0.0
    s = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    q = a / (Fraction(2) ** (e - 23))
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return s * float(Fraction(n) * Fraction(2) ** (e - 23))


def fma32(a, b, c):
    return f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def add32(a, b):
    return f32_round(Fraction(float(a)) + Fraction(float(b)))


def test_router_logit_fixed_order_exact(oracle):
    """The documented order (64 slots of fused multiply-adds over columns 4l+256i+c, then the
    xor butterfly) replayed with exact rational arithmetic reproduces the oracle's bits."""
    H, E = 512, 3
    W = CF.normal(CF.stream(90, 0, 0), E, H, 0.0, 0.05)
    x = CF.inputs(90, 1, H)[0]
    got = oracle.router_logits(W, x)[0]
    for e in range(E):
        v = []
        for l in range(64):
            acc = 0.0
            for i in range(H // 256):
                for c in range(4):
                    j = 4 * l + 256 * i + c
                    acc = fma32(W[e, j], x[j], acc)
            v.append(acc)
        for m in (32, 16, 8, 4, 2, 1):
            v = [add32(v[l], v[l ^ m]) for l in range(64)]
        assert np.float32(v[0]) == got[e]
        assert abs(float(got[e]) - float(W[e].astype(np.float64) @ x.astype(np.float64))) < 1e-5


def test_router_bias_added_after_reduction(oracle):
    H, E = 1024, 5
    W = CF.normal(CF.stream(91, 0, 0), E, H, 0.0, 0.02)
    x = CF.inputs(91, 2, H)
    b = np.arange(E, dtype=np.float32) * 0.5
    plain = oracle.router_logits(W, x)
    biased = oracle.router_logits(W, x, b, True)
    assert np.array_equal(biased, (plain + b).astype(np.float32))


# ------------------------------------------------------------------ formats
def row_of(kind, data):
    return np.frombuffer(bytes(data), np.uint8).copy()


def test_q8_0_textbook(oracle):
    rng = np.random.default_rng(1)
    for _ in range(20):
        d = float(np.float16(rng.uniform(1e-3, 1)))
        q = rng.integers(-128, 128, 32)
        blk = struct.pack("<H", f16(d)) + bytes(int(v) & 255 for v in q)
        got = [oracle.dequant_value(row_of(Q8_0, blk), Q8_0, j) for j in range(32)]
        assert np.array_equal(np.float32(got), np.float32(d) * q.astype(np.float32))


def test_q4_0_reference_fixture(oracle):
    g = GOLD["q4_0_fixture"]
    rows, cols = g["rows"], g["cols"]
    data = bytearray()
    for row in range(rows):
        for block in range(cols // 32):
            data += g["scale_f16_bits"].to_bytes(2, "little")
            for j in range(16):
                data.append((((row + block + j + 3) % 16) << 4) | ((row + block + j) % 16))
    m = Matrix(np.frombuffer(bytes(data), np.uint8).copy(), cols, rows, 1, Q4_0, 36)
    got = oracle.dequant_rows(m)
    r = np.arange(rows)[:, None]
    j = np.arange(cols)[None, :]
    nib = (r + j // 32 + j % 16 + np.where(j % 32 >= 16, 3, 0)) % 16
    assert np.array_equal(got, ((nib - 8.0) * 0.5).astype(np.float32))


def test_iq4_nl_values_and_layout(oracle):
    assert [oracle.dequant_value(row_of(IQ4_NL, struct.pack("<H", f16(1.0)) + bytes([v | (v << 4)] * 16)),
                                 IQ4_NL, 0) for v in range(16)] == \
        [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    blk = struct.pack("<H", f16(0.5)) + bytes([0x08] * 16)
    blk = bytearray(blk)
    blk[2 + 5] = 0xF8  # value 5 -> kvalues[8] = 1, value 21 -> kvalues[15] = 113
    vals = [oracle.dequant_value(row_of(IQ4_NL, blk), IQ4_NL, j) for j in range(32)]
    assert vals[5] == 0.5 and vals[21] == 56.5 and vals[16 + 4] == 0.5 * -127


def q4k_block(d, dmin, sc, mn, q):
    s = bytearray(12)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    qs = bytearray(128)
    for c in range(4):
        for i in range(32):
            qs[32 * c + i] = q[64 * c + i] | (q[64 * c + 32 + i] << 4)
    return struct.pack("<HH", f16(d), f16(dmin)) + bytes(s) + bytes(qs)


def test_q4_k_single_field_probes(oracle):
    """One non-zero nibble / one non-zero scale or min at a time: each field moves
    exactly the weights ggml's layout assigns to it (kernels/iq3_mix.metal:13-23)."""
    rng = np.random.default_rng(2)
    for trial in range(64):
        k = int(rng.integers(0, 256))
        g = k // 32
        sc = [0] * 8
        mn = [0] * 8
        sc[g] = int(rng.integers(1, 64))
        q = [0] * 256
        q[k] = int(rng.integers(1, 16))
        d, dmin = 0.25, 0.125
        blk = row_of(Q4_K, q4k_block(d, dmin, sc, mn, q))
        vals = np.array([oracle.dequant_value(blk, Q4_K, j) for j in range(256)])
        expect = np.zeros(256)
        expect[k] = d * sc[g] * q[k]
        assert np.array_equal(vals, expect), (k, sc[g], q[k])
    for g in range(8):  # min of group g subtracts dmin*m from exactly that group
        sc = [0] * 8
        mn = [0] * 8
        mn[g] = 37 + g
        blk = row_of(Q4_K, q4k_block(1.0, 0.5, sc, mn, [0] * 256))
        vals = np.array([oracle.dequant_value(blk, Q4_K, j) for j in range(256)])
        expect = np.zeros(256)
        expect[32 * g:32 * g + 32] = -0.5 * mn[g]
        assert np.array_equal(vals, expect)


def iq2xs_block(d, codes, scales):
    return struct.pack("<H", f16(d)) + struct.pack("<32H", *codes) + bytes(scales)


def _table(name):
    """A table of ingot_amd/csrc/codebooks.h (pinned by test_codebook_checksums_against_reference_text)."""
    import re
    src = open(os.path.join(os.path.dirname(HERE), "ingot_amd", "csrc", "codebooks.h")).read()
    m = re.search(name + r"\[(\d+)\]\s*=\s*\{(.*?)\};", src, re.S)
    return [int(v.rstrip("uUlL"), 0) for v in re.findall(r"-?0x[0-9a-fA-F]+[uUlL]*|-?\d+", m.group(2))]


def _ksign(i):
    return i | ((bin(i).count("1") & 1) << 7)


def test_iq2_xs_layout_probes(oracle):
    """IQ2_XS (kernels/iq3_mix.metal:25-30): the u16 code at 2 + 2 (4 g + l)
    drives values 32 g + 8 l .. + 7; value v is byte v of iq2xs_grid[code & 511],
    negated where bit v of the even-parity sign entry ksign(code >> 9) is set,
    times d (0.5 + nibble l / 2 of byte 66 + g) / 4. One random code and scale
    per probe, every other code 0 (grid entry 0, no signs): all 256 values are
    checked exactly, so a wrong code position, grid entry, byte order within an
    entry, sign bit or scale nibble fails."""
    grid = _table("ingot_iq2xs_grid")
    rng = np.random.default_rng(3)
    for trial in range(64):
        g, l = int(rng.integers(0, 8)), int(rng.integers(0, 4))
        gi, si, s = int(rng.integers(0, 512)), int(rng.integers(0, 128)), int(rng.integers(0, 16))
        codes = [0] * 32
        codes[4 * g + l] = gi | (si << 9)
        scales = [int(b) for b in rng.integers(0, 256, 8)]
        d = 0.75
        blk = row_of(IQ2_XS, iq2xs_block(d, codes, scales))
        vals = np.array([oracle.dequant_value(blk, IQ2_XS, j) for j in range(256)])
        for j in range(256):
            gg, ll, v = j // 32, (j % 32) // 8, j % 8
            code = codes[4 * gg + ll]
            sc = (scales[gg] >> (4 * (ll // 2))) & 15
            mag = (grid[code & 511] >> (8 * v)) & 255
            sign = -1.0 if _ksign(code >> 9) >> v & 1 else 1.0
            assert vals[j] == sign * d * (0.5 + sc) * 0.25 * mag, (trial, j)


def test_iq3_xxs_layout_probes(oracle):
    """IQ3_XXS (kernels/iq3_mix.metal:31-35): value v of sub-block l of group g is
    byte v % 4 of iq3xxs_grid[b[2 + 8 g + 2 l + v / 4]], negated where bit v of
    ksign((aux_g >> 7 l) & 127) is set, times d (0.5 + (aux_g >> 28)) / 2 with
    aux_g the u32 at 66 + 4 g. Two random grid bytes, sign index and scale per
    probe, every other grid byte 0: all 256 values are checked exactly."""
    grid = _table("ingot_iq3xxs_grid")
    rng = np.random.default_rng(4)
    for trial in range(64):
        g, l = int(rng.integers(0, 8)), int(rng.integers(0, 4))
        qs = [0] * 64
        qs[8 * g + 2 * l], qs[8 * g + 2 * l + 1] = int(rng.integers(0, 256)), int(rng.integers(0, 256))
        aux = [int(a) for a in rng.integers(0, 2 ** 32, 8, dtype=np.uint64)]
        d = 2.0
        blk = row_of(IQ3_XXS, struct.pack("<H", f16(d)) + bytes(qs) + struct.pack("<8I", *aux))
        vals = np.array([oracle.dequant_value(blk, IQ3_XXS, j) for j in range(256)])
        for j in range(256):
            gg, ll, v = j // 32, (j % 32) // 8, j % 8
            mag = (grid[qs[8 * gg + 2 * ll + v // 4]] >> (8 * (v % 4))) & 255
            sign = -1.0 if _ksign((aux[gg] >> (7 * ll)) & 127) >> v & 1 else 1.0
            assert vals[j] == sign * d * (0.5 + (aux[gg] >> 28)) * 0.5 * mag, (trial, j)


def test_codebook_checksums_against_reference_text():
    """The transcribed tables hash to the digests recorded from the reference's
    kernels/quant_tables.metal; re-derived from the text when the reference is mounted."""
    import re
    src = open(os.path.join(os.path.dirname(HERE), "ingot_amd", "csrc", "codebooks.h")).read()

    def table(text, name):
        m = re.search(name + r"\[(\d+)\]\s*=\s*\{(.*?)\};", text, re.S)
        return [int(v.rstrip("uUlL"), 0) for v in re.findall(r"-?0x[0-9a-fA-F]+[uUlL]*|-?\d+", m.group(2))]

    g2, g3, kv = table(src, "ingot_iq2xs_grid"), table(src, "ingot_iq3xxs_grid"), table(src, "ingot_kvalues_iq4nl")
    digests = GOLD["codebook_sha256"]
    assert hashlib.sha256(struct.pack("<512Q", *g2)).hexdigest() == digests["iq2xs_grid"]
    assert hashlib.sha256(struct.pack("<256I", *g3)).hexdigest() == digests["iq3xxs_grid"]
    assert hashlib.sha256(struct.pack("<16b", *kv)).hexdigest() == digests["kvalues_iq4nl"]
    assert all(b in (8, 25, 43) for v in g2 for b in ((v >> (8 * i)) & 255 for i in range(8)))
    assert all(b in (4, 12, 20, 28, 36, 44, 52, 62) for v in g3 for b in ((v >> (8 * i)) & 255 for i in range(4)))
    assert len(set(g2)) == 512 and len(set(g3)) == 256
    path = os.path.join(REFERENCE, "kernels", "quant_tables.metal")
    if os.path.exists(path):
        ref = open(path).read()
        assert table(ref, "iq2xs_grid") == g2
        assert table(ref, "iq3xxs_grid") == g3
        assert table(ref, "kvalues_iq4nl") == kv
        ks = table(ref, "ksigns_iq2xs")
        assert ks == [i | ((bin(i).count("1") & 1) << 7) for i in range(128)]


@pytest.mark.parametrize("kind,bound", [(Q4_0, 0.12), (Q8_0, 0.01), (Q4_K, 0.1), (IQ2_XS, 0.45), (IQ3_XXS, 0.3),
                                        (IQ4_NL, 0.1), (F32, 0.0)])
def test_quantize_dequantize_round_trip(oracle, kind, bound):
    w = CF.normal(CF.stream(92, kind, 0), 16, 512, 0.0, 0.02)
    m = CF.quantize(kind, w)
    assert oracle.validate(m)
    d = oracle.dequant_rows(m)
    err = np.sqrt(np.mean((d - w) ** 2)) / np.sqrt(np.mean(w ** 2))
    assert err <= bound


def test_geometry_and_validation_match_reference(oracle):
    table = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 8: (32, 34), 10: (256, 84), 12: (256, 144),
             13: (256, 176), 14: (256, 210), 16: (256, 66), 17: (256, 74), 18: (256, 98), 20: (32, 18),
             21: (256, 110), 22: (256, 82), 23: (256, 136), 29: (256, 56), 42: (64, 18)}
    for k in range(64):
        assert oracle.geometry(k) == table.get(k)


# ----------------------------------------------------------------- dispatch
def lcg(state):
    state = (state * 6364136223846793005 + 1442695040888963407) & ((1 << 64) - 1)
    return state, (state >> 11) / float(1 << 53)


def reference_plan(tokens, experts, top, skew):
    """src/expert_bench.rs:5-43 restated: skewed routes and the production tile layout."""
    state = GOLD["plan_generator"]["state"]
    groups = [[] for _ in range(experts)]
    ids = []
    for token in range(tokens):
        chosen = []
        while len(chosen) < top:
            state, u = lcg(state)
            e = int((u ** skew) * experts) % experts
            if e not in chosen:
                chosen.append(e)
        ids.extend(chosen)
        for k, e in enumerate(chosen):
            groups[e].append(token * top + k)
    pairs, tiles = [], []
    for expert, a in enumerate(groups):
        first = len(pairs)
        pairs.extend(a)
        for off in range(0, len(a), 32):
            nt = min(32, len(a) - off)
            tiles.append([expert, first + off, nt, int(nt >= 2)])
    return ids, pairs, tiles


@pytest.mark.parametrize("tokens,experts,top,skew", [(64, 128, 8, 1.0), (512, 128, 8, 3.0), (87, 512, 10, 2.0),
                                                     (5, 16, 4, 1.0)])
def test_dispatch_matches_reference_plan(oracle, tokens, experts, top, skew):
    ids, pairs, tiles = reference_plan(tokens, experts, top, skew)
    cap = (len(ids) + 31) // 32 + experts
    used, counts, first, opairs, inverse, otiles = oracle.dispatch(ids, experts, 32, cap)
    assert list(opairs) == pairs
    assert otiles[:used].tolist() == tiles
    assert not otiles[used:].any()
    assert all(opairs[inverse[p]] == p for p in range(len(ids)))


# ------------------------------------------------------------------- layer
def numpy_layer(spec, x, oracle):
    """The layer equation in float64 NumPy on the oracle's dequantised rows and its
    (separately pinned) fp32 routing: kernels/moe.metal:405-422, tools/check_rust_moe.py:55-75."""
    H, E, K, F = spec.hidden, spec.experts, spec.top_k, spec.ffn
    G = oracle.dequant_rows(spec.gate).reshape(E, F, H).astype(np.float64)
    U = oracle.dequant_rows(spec.up).reshape(E, F, H).astype(np.float64)
    D = oracle.dequant_rows(spec.down).reshape(E, H, F).astype(np.float64)
    logits = oracle.router_logits(spec.router, x, spec.router_bias, spec.router_bias is not None)
    out = np.zeros((x.shape[0], H))
    for t in range(x.shape[0]):
        ids, w = oracle.route_softmax(logits[t], K)
        xt = x[t].astype(np.float64)
        for e, wk in zip(ids, w):
            g, u = G[e] @ xt, U[e] @ xt
            out[t] += float(wk) * (D[e] @ (g / (1 + np.exp(-g)) * u))
        if spec.shared is not None:
            sg = oracle.dequant_rows(spec.shared[0]).astype(np.float64) @ xt
            su = oracle.dequant_rows(spec.shared[1]).astype(np.float64) @ xt
            s = oracle.dequant_rows(spec.shared[2]).astype(np.float64) @ (sg / (1 + np.exp(-sg)) * su)
            gate = 1.0
            if spec.shared_gate_vec is not None:
                gate = 1 / (1 + math.exp(-float(spec.shared_gate_vec.astype(np.float64) @ xt)))
            out[t] += gate * s
    return out


@pytest.mark.parametrize("shared", [False, True])
def test_layer_matches_numpy_equation(oracle, shared):
    spec = CF.make_layer(93, int(shared), 512, 6, 2, 256, Q4_K, Q8_0, bias="zipf", shared_ffn=256 if shared else 0,
                         shared_gated=shared)
    x = CF.inputs(93, 5, 512)
    st, out, ids, w = oracle.moe_forward(spec, x, oracle.F64)
    assert st == 0
    ref = numpy_layer(spec, x, oracle)
    assert np.abs(out - ref).max() < 1e-6 * max(1.0, np.abs(ref).max())


def test_layer_f32_agrees_with_f64_full_c0(oracle):
    spec = CF.c0_layer()
    x = CF.inputs(0, 2, 2048)
    _, o64, i64, w64 = oracle.moe_forward(spec, x, oracle.F64)
    _, o32, i32, w32 = oracle.moe_forward(spec, x, oracle.F32)
    assert np.array_equal(i64, i32) and np.array_equal(w64, w32)
    assert np.abs(o64 - o32).max() < 1e-5
    assert np.linalg.norm(o64 - o32) / np.linalg.norm(o64) < 1e-5


def test_layer_errors(oracle):
    spec = CF.make_layer(94, 0, 512, 4, 2, 256, Q4_K, Q4_K)
    x = CF.inputs(94, 1, 512)
    x[0, 3] = np.nan
    assert oracle.moe_forward(spec, x, oracle.F64)[0] == oracle.NONFINITE
    bad = LayerSpec(**{**spec.__dict__})
    bad.top_k = 5
    assert oracle.moe_forward(bad, CF.inputs(94, 1, 512), oracle.F64)[0] == oracle.INVALID
    # a finite input whose expert products overflow fp32: the output is rejected
    # (src/metal.rs:1575-1577); the routing, invariant under a positive scale, is still written
    x = CF.inputs(94, 2, 512)
    st, _, ids, _ = oracle.moe_forward(spec, x, oracle.F64)
    assert st == oracle.OK
    for prec in (oracle.F64, oracle.F32):
        st, out, ids2, _ = oracle.moe_forward(spec, x * np.float32(1e25), prec)
        assert st == oracle.NONFINITE and not np.isfinite(out).all()
        assert np.array_equal(ids, ids2)


def test_rmsnorm_residual_equation(oracle):
    spec = CF.make_layer(95, 0, 512, 4, 2, 256, Q4_K, Q4_K, norm=True)
    x = CF.inputs(95, 3, 512) * 3.0
    st, out, ids, w = oracle.moe_forward(spec, x, oracle.F64)
    assert st == 0
    xn = x / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6) * spec.norm_gain
    plain = LayerSpec(**{**spec.__dict__})
    plain.norm_gain = None
    st2, moe, ids2, _ = oracle.moe_forward(plain, xn.astype(np.float32), oracle.F64)
    assert st2 == 0
    # xn here is rounded once from float64; the layer's fixed-order fp32 norm may differ in the
    # last ulp, which moves the output far less than the tolerance (ids agree on this input).
    assert np.array_equal(ids, ids2)
    assert np.abs(out - (x + moe)).max() < 1e-4


# ------------------------------------------------------------------- synth
def test_synth_streams_are_deterministic_and_thread_independent():
    import ctypes
    from ingot_amd import _native as N
    lib = N.synth_lib()
    a = np.empty((37, 100), np.float32)
    b = np.empty((37, 100), np.float32)
    lib.ingot_synth_normal(123, 37, 100, 0.0, 1.0, a.ctypes.data, 1)
    lib.ingot_synth_normal(123, 37, 100, 0.0, 1.0, b.ctypes.data, 7)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 0.05 and abs(a.std() - 1) < 0.05
    m1 = CF.synth_matrix(Q4_K, 77, 3, 8, 512)
    m2 = CF.synth_matrix(Q4_K, 77, 3, 8, 512)
    assert np.array_equal(m1.data, m2.data)
    x = np.array([1.0, 1.00390625, 1.005859375, -3.0e38, 1e-40], np.float32)
    r = CF.round_bf16(x)
    assert list(r[:3]) == [1.0, 1.0, 1.0078125]
    with np.errstate(over="ignore"):
        for v in np.linspace(-70000, 70000, 1001).astype(np.float32):
            assert lib.ingot_f32_to_f16(float(v)) == int(np.float16(v).view(np.uint16))
        for v in (1e-8, 6e-8, 3e-5, 6.1e-5, 65504.0, 65520.0):
            assert lib.ingot_f32_to_f16(v) == int(np.float16(np.float32(v)).view(np.uint16)), v
