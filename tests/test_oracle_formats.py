"""CPU pins of the oracle's decoders for the formats beyond the graded
configurations: Q2_K, Q5_K, Q6_K, IQ2_XXS, IQ2_S, IQ3_S, IQ4_XS, IQ1_M, BF16
and Q2_0 (kernels/moe.metal:17-89, kernels/iq3_mix.metal:19-23).

No external known-answer vectors exist for these formats in the reference, so
each decoder is pinned by single-field probes: one non-zero quant, index,
sign, scale or min at a time, which must move exactly the weights the
reference's layout assigns to it, by the amount its formula gives; by
special cases that reduce to an already pinned format (Q5_K with no fifth
bits is Q4_K); and by the codebooks' checksums and value sets.
"""
import hashlib
import json
import os
import re
import struct

import numpy as np
import pytest

from ingot_amd.moe import BF16, IQ1_M, IQ2_S, IQ2_XXS, IQ3_S, IQ4_XS, Q2_0, Q2_K, Q4_K, Q5_K, Q6_K

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "reference_known_answers.json")))
KVALUES = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
SRC = open(os.path.join(os.path.dirname(HERE), "ingot_amd", "csrc", "codebooks.h")).read()


def table(text, name):
    m = re.search(name + r"\[(\d+)\]\s*=\s*\{(.*?)\};", text, re.S)
    return [int(v.rstrip("uUlL"), 0) for v in re.findall(r"-?0x[0-9a-fA-F]+[uUlL]*|-?\d+", m.group(2))]


GRID = {n: table(SRC, "ingot_" + n) for n in ("iq2xxs_grid", "iq2s_grid", "iq3s_grid", "iq1s_grid")}


def f16(x):
    return int(np.float16(x).view(np.uint16))


def decode(oracle, kind, blk, n=256):
    row = np.frombuffer(bytes(blk), np.uint8).copy()
    return np.array([oracle.dequant_value(row, kind, j) for j in range(n)])


def ksign(i):
    return i | ((bin(i).count("1") & 1) << 7)


# ---------------------------------------------------------------- codebooks
def test_new_codebooks_checksums_and_value_sets():
    d = GOLD["codebook_sha256"]
    packs = {"iq2xxs_grid": "<256Q", "iq2s_grid": "<1024Q", "iq3s_grid": "<512I", "iq1s_grid": "<2048Q"}
    for name, fmt in packs.items():
        assert hashlib.sha256(struct.pack(fmt, *GRID[name])).hexdigest() == d[name], name
        assert len(set(GRID[name])) == len(GRID[name])
    byts = lambda vals, n: {(v >> (8 * i)) & 255 for v in vals for i in range(n)}  # noqa: E731
    assert byts(GRID["iq2xxs_grid"], 8) <= {8, 25, 43} and byts(GRID["iq2s_grid"], 8) <= {8, 25, 43}
    assert byts(GRID["iq3s_grid"], 4) <= set(range(1, 16, 2))
    assert byts(GRID["iq1s_grid"], 8) <= {0xff, 0, 1}
    path = "/root/reference/kernels/quant_tables.metal"
    if os.path.exists(path):
        ref = open(path).read()
        for name in packs:
            assert table(ref, name) == GRID[name], name


# ------------------------------------------------------------------ K-quants
def q4k_scales(sc, mn):
    s = bytearray(12)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(s)


def q5k_block(d, dmin, sc, mn, q):
    """q: 256 five-bit values; nibbles as Q4_K's @48, fifth bit of value k in
    bit k//32 of byte 16 + k%32."""
    qh = bytearray(32)
    qs = bytearray(128)
    for k in range(256):
        qh[k % 32] |= ((q[k] >> 4) & 1) << (k // 32)
        c, i, hi = k // 64, k % 32, (k % 64) // 32
        qs[32 * c + i] |= (q[k] & 15) << (4 * hi)
    return struct.pack("<HH", f16(d), f16(dmin)) + q4k_scales(sc, mn) + bytes(qh) + bytes(qs)


def test_q5_k_probes_and_q4_k_special_case(oracle):
    rng = np.random.default_rng(10)
    for _ in range(48):
        k = int(rng.integers(0, 256))
        sc, mn, q = [0] * 8, [0] * 8, [0] * 256
        sc[k // 32] = int(rng.integers(1, 64))
        q[k] = int(rng.integers(1, 32))
        vals = decode(oracle, Q5_K, q5k_block(0.25, 0.125, sc, mn, q))
        expect = np.zeros(256)
        expect[k] = 0.25 * sc[k // 32] * q[k]
        assert np.array_equal(vals, expect), (k, q[k])
    # no fifth bits: the block decodes as the Q4_K block with the same header and nibbles
    sc = [int(v) for v in rng.integers(0, 64, 8)]
    mn = [int(v) for v in rng.integers(0, 64, 8)]
    q = [int(v) for v in rng.integers(0, 16, 256)]
    b5 = q5k_block(0.5, 0.25, sc, mn, q)
    b4 = b5[:16] + b5[48:]
    assert np.array_equal(decode(oracle, Q5_K, b5), decode(oracle, Q4_K, b4))


def q6k_block(d, sc, q):
    """q: 256 six-bit values, sc: 16 int8 scales (kernels/moe.metal:22-28)."""
    ql, qh = bytearray(128), bytearray(64)
    for k in range(256):
        n, l, t = k // 128, k % 32, (k % 128) // 32
        ql[64 * n + l + 32 * (t % 2)] |= (q[k] & 15) << (4 if t >= 2 else 0)
        qh[32 * n + l] |= (q[k] >> 4) << (2 * t)
    return bytes(ql) + bytes(qh) + struct.pack("<16b", *sc) + struct.pack("<H", f16(d))


def test_q6_k_probes(oracle):
    rng = np.random.default_rng(11)
    for _ in range(64):
        k = int(rng.integers(0, 256))
        sc = [0] * 16
        n, l, t = k // 128, k % 32, (k % 128) // 32
        s = int(rng.integers(-128, 128))
        sc[8 * n + l // 16 + 2 * t] = s
        q = [32] * 256  # q = 32 decodes to 0
        q[k] = int(rng.integers(0, 64))
        vals = decode(oracle, Q6_K, q6k_block(0.5, sc, q))
        expect = np.zeros(256)
        expect[k] = 0.5 * s * (q[k] - 32)
        assert np.array_equal(vals, expect), (k, s, q[k])
    # every value of the scale's 16-group, and no other, takes that scale
    for j in range(16):
        sc = [0] * 16
        sc[j] = 3
        vals = decode(oracle, Q6_K, q6k_block(1.0, sc, [0] * 256))
        hit = np.nonzero(vals)[0]
        n, r = j // 8, j % 8  # scale 8n + l/16 + 2t
        t, half = r // 2, r % 2
        first = 128 * n + 32 * t + 16 * half
        assert list(hit) == list(range(first, first + 16)) and np.all(vals[hit] == -96.0)


def q2k_block(d, dmin, sc, q):
    """sc: 16 bytes (scale | min << 4), q: 256 two-bit values."""
    qs = bytearray(64)
    for k in range(256):
        qs[(k // 128) * 32 + k % 32] |= q[k] << (2 * ((k % 128) // 32))
    return bytes(sc) + bytes(qs) + struct.pack("<HH", f16(d), f16(dmin))


def test_q2_k_probes(oracle):
    rng = np.random.default_rng(12)
    for _ in range(64):
        k = int(rng.integers(0, 256))
        sc = [0] * 16
        s = int(rng.integers(1, 16))
        sc[k // 16] = s
        q = [0] * 256
        q[k] = int(rng.integers(1, 4))
        vals = decode(oracle, Q2_K, q2k_block(0.5, 0.25, sc, q))
        expect = np.zeros(256)
        expect[k] = 0.5 * s * q[k]
        assert np.array_equal(vals, expect)
    for j in range(16):
        sc = [0] * 16
        sc[j] = 5 << 4  # min only: -dmin * 5 on exactly that 16-group
        vals = decode(oracle, Q2_K, q2k_block(1.0, 0.5, sc, [3] * 256))
        expect = np.zeros(256)
        expect[16 * j:16 * j + 16] = -2.5
        assert np.array_equal(vals, expect)


# ------------------------------------------------------------ IQ codebooks
def test_iq2_xxs_probes(oracle):
    rng = np.random.default_rng(13)
    for _ in range(48):
        g, l = int(rng.integers(0, 8)), int(rng.integers(0, 4))
        gi, si, s = int(rng.integers(0, 256)), int(rng.integers(0, 128)), int(rng.integers(0, 16))
        groups = bytearray(64)
        groups[8 * g + l] = gi
        aux = (si << (7 * l)) | (s << 28)
        groups[8 * g + 4:8 * g + 8] = struct.pack("<I", aux)
        vals = decode(oracle, IQ2_XXS, struct.pack("<H", f16(2.0)) + bytes(groups))
        sub = vals[32 * g + 8 * l:32 * g + 8 * l + 8]
        db = 2.0 * (0.5 + s) * 0.25
        for v in range(8):
            mag = (GRID["iq2xxs_grid"][gi] >> (8 * v)) & 255
            assert sub[v] == (-1 if ksign(si) >> v & 1 else 1) * db * mag
        # the group's other sub-blocks use index 0 and sign index 0 with the same scale
        rest = np.delete(vals[32 * g:32 * g + 32], range(8 * l, 8 * l + 8))
        assert np.all(rest == db * 8)


def test_iq2_s_probes(oracle):
    rng = np.random.default_rng(14)
    for _ in range(48):
        g, l = int(rng.integers(0, 8)), int(rng.integers(0, 4))
        idx, sg, s = int(rng.integers(0, 1024)), int(rng.integers(0, 256)), int(rng.integers(0, 16))
        b = bytearray(82)
        b[0:2] = struct.pack("<H", f16(1.0))
        b[2 + 4 * g + l] = idx & 255
        b[66 + g] = (idx >> 8) << (2 * l)
        b[34 + 4 * g + l] = sg
        b[74 + g] = s << (4 * (l // 2))
        vals = decode(oracle, IQ2_S, b)
        sub = vals[32 * g + 8 * l:32 * g + 8 * l + 8]
        for v in range(8):
            mag = (GRID["iq2s_grid"][idx] >> (8 * v)) & 255
            assert sub[v] == (-1 if sg >> v & 1 else 1) * (0.5 + s) * 0.25 * mag


def test_iq3_s_probes(oracle):
    rng = np.random.default_rng(15)
    for _ in range(48):
        g, j = int(rng.integers(0, 8)), int(rng.integers(0, 8))  # grid entry j: values 4j..4j+3
        idx, sg, s = int(rng.integers(0, 512)), int(rng.integers(0, 256)), int(rng.integers(0, 16))
        b = bytearray(110)
        b[0:2] = struct.pack("<H", f16(0.5))
        b[2 + 8 * g + j] = idx & 255
        b[66 + g] = (idx >> 8) << j
        b[74 + 4 * g + j // 2] = sg
        b[106 + g // 2] = s << (4 * (g % 2))
        vals = decode(oracle, IQ3_S, b)
        sub = vals[32 * g + 4 * j:32 * g + 4 * j + 4]
        for v in range(4):
            mag = (GRID["iq3s_grid"][idx] >> (8 * v)) & 255
            sign = -1 if sg >> (4 * (j % 2) + v) & 1 else 1
            assert sub[v] == sign * 0.5 * (1 + 2 * s) * mag


def test_iq4_xs_probes(oracle):
    rng = np.random.default_rng(16)
    for _ in range(48):
        g, v = int(rng.integers(0, 8)), int(rng.integers(0, 32))
        scale, q = int(rng.integers(0, 64)), int(rng.integers(0, 16))
        b = bytearray(136)
        b[0:2] = struct.pack("<H", f16(0.5))
        b[2:4] = struct.pack("<H", (scale >> 4) << (2 * g))
        b[4 + g // 2] = (scale & 15) << (4 * (g % 2))
        for i in range(16):
            b[8 + 16 * g + i] = 0x88  # kvalues[8] = 1 everywhere in the group
        b[8 + 16 * g + v % 16] = (q << 4 * (v // 16)) | (8 << 4 * (1 - v // 16))
        vals = decode(oracle, IQ4_XS, b)
        grp = vals[32 * g:32 * g + 32]
        expect = np.full(32, 0.5 * (scale - 32) * 1.0)
        expect[v] = 0.5 * (scale - 32) * KVALUES[q]
        assert np.array_equal(grp, expect)
        assert np.all(np.delete(vals, range(32 * g, 32 * g + 32)) == 0.5 * -32 * KVALUES[0])


def iq1m_block(d, qs, qh, scales):
    """scales: 16 three-bit values (per 16 weights) packed 4 per u16 word with
    the fp16 d in the words' top nibbles."""
    words = [0] * 4
    for i, s in enumerate(scales):
        g, h = i // 2, i % 2  # group g, half h
        words[g // 2] |= s << (6 * (g % 2) + 3 * h)
    bits = f16(d)
    for w in range(4):
        words[w] |= ((bits >> (4 * w)) & 15) << 12
    return bytes(qs) + bytes(qh) + struct.pack("<4H", *words)


def test_iq1_m_probes(oracle):
    rng = np.random.default_rng(17)
    for _ in range(48):
        g, l = int(rng.integers(0, 8)), int(rng.integers(0, 4))
        idx, neg, s = int(rng.integers(0, 2048)), int(rng.integers(0, 2)), int(rng.integers(0, 8))
        qs, qh, scales = bytearray(32), bytearray(16), [0] * 16
        qs[4 * g + l] = idx & 255
        qh[2 * g + l // 2] = ((idx >> 8) | (neg << 3)) << (4 * (l % 2))
        scales[2 * g + l // 2] = s
        vals = decode(oracle, IQ1_M, iq1m_block(0.5, qs, qh, scales))
        sub = vals[32 * g + 8 * l:32 * g + 8 * l + 8]
        delta = -0.125 if neg else 0.125
        for v in range(8):
            grid = int(np.uint8((GRID["iq1s_grid"][idx] >> (8 * v)) & 255).view(np.int8))
            assert sub[v] == np.float32(0.5 * (2 * s + 1)) * np.float32(grid + delta)
    # d round-trips through the four top nibbles
    for d in (1.0, 0.0009765625, 3.5, -2.0):
        vals = decode(oracle, IQ1_M, iq1m_block(d, bytes(32), bytes(16), [0] * 16))
        grid0 = int(np.uint8(GRID["iq1s_grid"][0] & 255).view(np.int8))
        assert vals[0] == np.float32(d) * np.float32(grid0 + 0.125)


def test_q2_0_and_bf16(oracle):
    rng = np.random.default_rng(18)
    for _ in range(32):
        k, c = int(rng.integers(0, 64)), int(rng.integers(0, 4))
        b = bytearray(18)
        b[0:2] = struct.pack("<H", f16(0.75))
        for i in range(16):
            b[2 + i] = 0x55  # code 1 everywhere: 0
        b[2 + k // 4] = (0x55 & ~(3 << 2 * (k % 4))) | (c << 2 * (k % 4))
        vals = decode(oracle, Q2_0, b, 64)
        expect = np.zeros(64)
        expect[k] = 0.75 * (c - 1)
        assert np.array_equal(vals, expect)
    x = np.array([1.0, -2.5, 3.140625, 1e-30, -0.0], np.float32)
    bf = (x.view(np.uint32) >> 16).astype("<u2")
    got = decode(oracle, BF16, bf.tobytes(), len(x))
    assert np.array_equal(got.astype(np.float32), (bf.astype(np.uint32) << 16).view(np.float32))
