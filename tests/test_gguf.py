"""CPU tests of the GGUF reader (ingot_amd/gguf.py) and the moe-layer
command's error contract (ingot_amd/moe_layer.py).

The first two tests restate the reference reader's own tests on a file built
byte by byte (src/gguf.rs:493-586); the rest cover each directory check of
src/gguf.rs:117-203, the shard rules of :205-271, the expert slabs of
:434-460, and src/main.rs:255-325 up to the point where the GPU is needed.
"""
import math
import os
import struct

import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd import gguf as G
from ingot_amd.moe import IQ2_XS, Q4_K, Q8_0, ROUTE_SIGMOID, InvalidData
from ingot_amd.moe_layer import USAGE, main, rust_f32


def text(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def kv(key, kind, payload: bytes) -> bytes:
    return text(key) + struct.pack("<I", kind) + payload


def header(tensors, metadata=(), nt=None, nm=None, version=3, magic=0x46554747) -> bytes:
    """GGUF header bytes: general.architecture = "fixture", then the encoded
    metadata entries (kv(...)) and tensors (name, dims, kind, offset),
    written field by field."""
    h = struct.pack("<IIQQ", magic, version, len(tensors) if nt is None else nt,
                    len(metadata) + 1 if nm is None else nm)
    h += kv("general.architecture", G.T_STRING, text("fixture"))
    for m in metadata:
        h += m
    for name, dims, kind, off in tensors:
        h += text(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        h += struct.pack("<IQ", kind, off)
    return h


def pad(b: bytes, a: int = 32) -> bytes:
    return b + b"\0" * ((-len(b)) % a)


def f32s(*v) -> bytes:
    return b"".join(struct.pack("<f", x) for x in v)


# -------------------------------------------------- the reference's own tests
def test_truncated_header_and_unknown_geometry(tmp_path):
    """src/gguf.rs:493-502."""
    p = tmp_path / "t.gguf"
    p.write_bytes(b"GGUF\x03\0\0\0")
    with pytest.raises(InvalidData):
        G.Gguf.open(p)
    with pytest.raises(InvalidData):
        G.geometry(19)


def test_positional_reads_report_truncation_after_validation(tmp_path):
    """src/gguf.rs:503-586: one 2x2 F32 tensor 'weight' = [[1, 2], [3, 4]]."""
    p = tmp_path / "short.gguf"
    h = pad(header([("weight", [2, 2], 0, 0)]))
    payload = len(h)
    data = h + f32s(1, 2, 3, 4)
    with open(p, "xb") as f:
        f.write(data)
    g = G.Gguf.open(p)
    t = g.tensor("weight")
    assert (t.dims, t.kind, t.offset, t.stride, t.bytes) == ([2, 2], 0, payload, 8, 16)
    mapped = g.map_tensor(t)
    assert bytes(mapped) == data[payload:]
    del mapped  # never truncate a file with live mappings
    assert g.rows("weight", [1]).data.tobytes() == f32s(3, 4)
    before = g.bytes_read
    assert g.rows("weight", [1, 0, 1, 0]).data.tobytes() == f32s(3, 4, 1, 2, 3, 4, 1, 2)
    assert g.bytes_read - before == 32
    assert g.row_read_time > 0
    before = g.bytes_read
    with pytest.raises(InvalidData):
        g.rows("weight", [])
    with pytest.raises(InvalidData):
        g.rows("weight", [0, 2])
    assert g.bytes_read == before
    os.truncate(p, payload + 10)
    with pytest.raises(EOFError):
        g.map_tensor(g.tensor("weight"))
    with pytest.raises(EOFError):
        g.rows("weight", [1])
    before, elapsed = g.bytes_read, g.row_read_time
    with pytest.raises(EOFError):
        g.rows("weight", [0, 1, 0, 1])
    # Every row is attempted before the error; the two whole rows count.
    assert g.bytes_read - before == 16
    assert g.row_read_time > elapsed
    g.close()


# ------------------------------------------------------------ directory checks
def test_metadata_types(tmp_path):
    """src/gguf.rs:87-116: every width of integer reads unsigned, F32 and F64
    as float, arrays of any element type but arrays."""
    meta = [
        kv("u8", G.T_U8, b"\xfe"), kv("i8", G.T_I8, b"\xff"), kv("b", G.T_BOOL, b"\x01"),
        kv("u16", G.T_U16, struct.pack("<H", 65535)), kv("i16", G.T_I16, struct.pack("<h", -2)),
        kv("u32", G.T_U32, struct.pack("<I", 7)), kv("i32", G.T_I32, struct.pack("<i", -1)),
        kv("u64", G.T_U64, struct.pack("<Q", 2 ** 63)), kv("i64", G.T_I64, struct.pack("<q", -1)),
        kv("f32", G.T_F32, struct.pack("<f", 0.1)), kv("f64", G.T_F64, struct.pack("<d", 1e300)),
        kv("s", G.T_STRING, text("héllo")),
        kv("ai", G.T_ARRAY, struct.pack("<IQ", G.T_U16, 3) + struct.pack("<3H", 1, 2, 3)),
        kv("as", G.T_ARRAY, struct.pack("<IQ", G.T_STRING, 2) + text("a") + text("b")),
        kv("af", G.T_ARRAY, struct.pack("<IQ", G.T_F32, 1) + f32s(2.5)),
        kv("ae", G.T_ARRAY, struct.pack("<IQ", G.T_U8, 0)),
    ]
    p = tmp_path / "m.gguf"
    p.write_bytes(header([], meta))
    g = G.Gguf.open(p)
    assert g.architecture == "fixture"
    assert [g.integer(k) for k in ("u8", "i8", "b", "u16", "i16", "u32", "i32", "u64", "i64")] == \
        [254, 255, 1, 65535, 65534, 7, 2 ** 32 - 1, 2 ** 63, 2 ** 64 - 1]
    assert g.float("f32") == float(np.float32(0.1))
    with pytest.raises(InvalidData, match="missing float: f64"):
        g.float("f64")  # finite as f64, infinite as f32
    assert g.optional_float("f64") is None and g.optional_float("u8") is None
    with pytest.raises(InvalidData):
        g.integer("f32")
    assert g.optional_integer("s") is None and g.optional_integer("nope") is None
    assert g.string("s") == "héllo" and g.optional_string("u8") is None
    assert g.integers("ai") == [1, 2, 3] and g.strings("as") == ["a", "b"]
    assert g.integers("ae") == [] and g.array("af") == [2.5]
    with pytest.raises(InvalidData):
        g.integers("as")
    with pytest.raises(InvalidData):
        g.strings("ai")
    with pytest.raises(InvalidData, match="missing array: s"):
        g.array("s")


BAD_DIRECTORIES = {
    "magic": lambda: header([], magic=0x46554748),
    "version 2": lambda: header([], version=2),
    "duplicate metadata": lambda: header([], [kv("general.architecture", G.T_STRING, text("x"))]),
    "nested array": lambda: header([], [kv("a", G.T_ARRAY, struct.pack("<IQ", G.T_ARRAY, 0))]),
    "unknown metadata type": lambda: header([], [kv("a", 13, b"\0" * 8)]),
    "truncated string": lambda: header([], [kv("s", G.T_STRING, struct.pack("<Q", 1000) + b"ab")]),
    "truncated array": lambda: header([], [kv("a", G.T_ARRAY, struct.pack("<IQ", G.T_U8, 1 << 40))]),
    "missing tensor record": lambda: header([], nt=1),
    "alignment 48": lambda: header([], [kv("general.alignment", G.T_U32, struct.pack("<I", 48))]),
    "alignment 0": lambda: header([], [kv("general.alignment", G.T_U32, struct.pack("<I", 0))]),
    "alignment float": lambda: header([], [kv("general.alignment", G.T_F32, f32s(32.0))]),
    "rank 0": lambda: pad(header([("w", [], 0, 0)])) + f32s(1),
    "rank 5": lambda: pad(header([("w", [1, 1, 1, 1, 1], 0, 0)])) + f32s(1),
    "zero dim": lambda: pad(header([("w", [4, 0], 0, 0)])),
    "partial block": lambda: pad(header([("w", [255], Q4_K, 0)])) + b"\0" * 144,
    "unaligned offset": lambda: pad(header([("w", [1], 0, 4)])) + f32s(0, 1),
    "unknown tensor type": lambda: pad(header([("w", [1], 19, 0)])) + b"\0" * 64,
    "duplicate tensor": lambda: pad(header([("w", [1], 0, 0), ("w", [1], 0, 32)])) + b"\0" * 64,
    "beyond file": lambda: pad(header([("w", [4], 0, 0)])) + f32s(1, 2, 3),
    "overlap": lambda: pad(header([("a", [16], 0, 0), ("b", [8], 0, 32)])) + b"\0" * 64,
    "no architecture": lambda: struct.pack("<IIQQ", 0x46554747, 3, 0, 0),
}


@pytest.mark.parametrize("case", sorted(BAD_DIRECTORIES))
def test_directory_checks(tmp_path, case):
    """Each check of src/gguf.rs:117-203 and :205-213 rejects its case."""
    p = tmp_path / "bad.gguf"
    p.write_bytes(BAD_DIRECTORIES[case]())
    with pytest.raises(InvalidData):
        G.Gguf.open(p)


def test_alignment_and_adjacent_tensors(tmp_path):
    """Data start rounds up to general.alignment; offsets are relative to it;
    touching tensor ranges do not overlap."""
    for align in (1, 64, 4096):
        p = tmp_path / f"a{align}.gguf"
        h = header([("a", [16], 0, 0), ("b", [2, 1], 0, 64 if align <= 64 else align)],
                   [kv("general.alignment", G.T_U64, struct.pack("<Q", align))])
        start = len(pad(h, align))
        body = f32s(*range(16)) + b"\0" * ((64 if align <= 64 else align) - 64) + f32s(7, 8)
        p.write_bytes(pad(h, align) + body)
        with G.Gguf.open(p) as g:
            assert g.tensor("a").offset == start and g.tensor("a").offset % align == 0
            assert g.rows("b", [0]).data.tobytes() == f32s(7, 8)
            assert g.rows("a", [0]).data.tobytes() == f32s(*range(16))


def test_writer_round_trip(tmp_path):
    p = str(tmp_path / "w.gguf")
    q = CF.synth_matrix(Q8_0, 7, 3, 4, 64)
    G.write_gguf(p, {"general.architecture": "x", "k.i": 5, "k.f": 0.5, "k.s": "v", "k.a": [1, 2],
                     "k.neg": (G.T_I32, -3)},
                 [("q", [64, 4, 3], Q8_0, q.data), ("f", [3], 0, f32s(1, 2, 3))], alignment=64)
    with pytest.raises(FileExistsError):
        G.write_gguf(p, {"general.architecture": "x"}, [])
    with G.Gguf.open(p) as g:
        assert g.integer("k.i") == 5 and g.float("k.f") == 0.5 and g.string("k.s") == "v"
        assert g.integers("k.a") == [1, 2] and g.integer("k.neg") == 2 ** 32 - 3
        t = g.tensor("q")
        assert (t.stride, t.bytes, t.offset % 64) == (68, 68 * 12, 0)
        assert bytes(g.map_tensor(t)) == q.data.tobytes()


# ------------------------------------------------------------- expert slabs
def test_matrix_expert_slabs(tmp_path):
    """src/gguf.rs:434-460: shape must equal dims; experts in the given order,
    repeats allowed; each slab is stride x rows bytes."""
    E, F, H = 5, 8, 256
    q = CF.synth_matrix(Q4_K, 11, E, F, H)
    p = str(tmp_path / "m.gguf")
    G.write_gguf(p, {"general.architecture": "x"}, [("w", [H, F, E], Q4_K, q.data), ("v", [H], 0, np.ones(H, "<f4"))])
    with G.Gguf.open(p) as g:
        before = g.bytes_read
        m = g.matrix("w", [H, F, E], [3, 1, 3])
        assert (m.cols, m.rows, m.count, m.kind, m.stride) == (H, F, 3, Q4_K, 144)
        assert m.data.tobytes() == q.select([3, 1, 3]).data.tobytes()
        assert g.bytes_read - before == 3 * F * 144
        v = g.matrix("w", [H, F, E], range(1, 4), copy=False)
        assert isinstance(v.data, np.memmap) and v.data.tobytes() == q.select([1, 2, 3]).data.tobytes()
        assert g.matrix("w", [H, F, E], [4, 2], copy=False).data.tobytes() == q.select([4, 2]).data.tobytes()
        vec = g.matrix("v", [H], [0])
        assert (vec.cols, vec.rows, vec.count) == (H, 1, 1)
        with pytest.raises(InvalidData, match=r"w: expected \[256, 8, 4\], found \[256, 8, 5\]"):
            g.matrix("w", [H, F, 4], [0])
        for bad in ([], [5], [-1]):
            with pytest.raises(InvalidData):
                g.matrix("w", [H, F, E], bad)
        with pytest.raises(InvalidData, match="missing tensor: nope"):
            g.matrix("nope", [H], [0])
        r = g.rows("w", [F * E - 1, 0])
        assert (r.rows, r.count) == (2, 1)
        assert r.data.tobytes() == q.data[-144:].tobytes() + q.data[:144].tobytes()


def test_ffn_weights_names_and_shapes(tmp_path):
    """src/lib.rs:62-88: blk.L.ffn_{gate,up,down}_{exps|shexp}.weight."""
    spec = CF.make_layer(50, 0, 512, 6, 2, 256, IQ2_XS, Q8_0, shared_ffn=512, shared_gate_kind=Q8_0,
                         shared_down_kind=Q8_0, shared_gated=True)
    p = str(tmp_path / "l.gguf")
    G.write_gguf(p, G.layer_metadata(spec, "qwen4exp", 3), G.layer_tensors(spec, 2))
    with G.Gguf.open(p) as g:
        gate, up, down = G.ffn_weights(g, 2, 512, 256, 6, [5, 0], False)
        for got, want in ((gate, spec.gate), (up, spec.up), (down, spec.down)):
            assert got.data.tobytes() == want.select([5, 0]).data.tobytes()
            assert (got.cols, got.rows, got.count, got.kind) == (want.cols, want.rows, 2, want.kind)
        sg, su, sd = G.ffn_weights(g, 2, 512, 512, 1, [0], True)
        assert sd.data.tobytes() == spec.shared[2].data.tobytes() and (sd.cols, sd.rows) == (512, 512)
        with pytest.raises(InvalidData):
            G.ffn_weights(g, 2, 512, 128, 6, [0], False)  # wrong expert hidden size
        with pytest.raises(InvalidData):
            G.ffn_weights(g, 1, 512, 256, 6, [0], False)  # no such layer


@pytest.mark.parametrize("norm", [False, True])
def test_layer_spec_round_trip(tmp_path, norm):
    """layer_spec reads back what layer_tensors/layer_metadata wrote: every
    byte of every matrix, the router, bias, shared gate and (norm=True) gain."""
    spec = CF.make_layer(51, 1, 512, 8, 3, 256, Q4_K, Q8_0, routing=ROUTE_SIGMOID, route_scale=2.5,
                         bias="uniform", shared_ffn=256, shared_gated=True, norm=True)
    p = str(tmp_path / "l.gguf")
    G.write_gguf(p, G.layer_metadata(spec, "glmish", 2), G.layer_tensors(spec, 1))
    with G.Gguf.open(p) as g:
        got = G.layer_spec(g, 1, norm=norm)
        assert (got.hidden, got.experts, got.top_k, got.routing, got.route_scale) == (512, 8, 3, ROUTE_SIGMOID, 2.5)
        assert np.array_equal(got.router, spec.router) and np.array_equal(got.router_bias, spec.router_bias)
        assert np.array_equal(got.shared_gate_vec, spec.shared_gate_vec)
        for a, b in zip((got.gate, got.up, got.down) + got.shared, (spec.gate, spec.up, spec.down) + spec.shared):
            assert (a.cols, a.rows, a.count, a.kind, a.stride) == (b.cols, b.rows, b.count, b.kind, b.stride)
            assert np.array_equal(np.asarray(a.data), b.data)
        if norm:
            assert np.array_equal(got.norm_gain, spec.norm_gain) and got.norm_eps == np.float32(spec.norm_eps)
        else:
            assert got.norm_gain is None
        with pytest.raises(InvalidData, match="layer out of range"):
            G.layer_spec(g, 2)


# -------------------------------------------------------------------- shards
def shard_model(tmp_path, shards=3):
    spec = CF.make_layer(52, 0, 256, 4, 2, 256, Q8_0, Q8_0)
    meta = G.layer_metadata(spec, "qwen4exp", 1)
    tensors = G.layer_tensors(spec, 0)
    return spec, meta, tensors, G.write_split(str(tmp_path / "model"), meta, tensors, shards)


def test_split_model_opens_from_first_shard(tmp_path):
    """src/gguf.rs:221-268: NAME-0000k-of-0000n.gguf, consistent split keys,
    every tensor once, split.tensors.count tensors in all."""
    spec, meta, tensors, paths = shard_model(tmp_path)
    with G.Gguf.open(paths[0]) as g:
        assert len(g.files) == 3 and sorted(g.tensors) == sorted(t[0] for t in tensors)
        assert {g.tensors[t[0]].shard for t in tensors} == {0, 1, 2}
        got = G.layer_spec(g, 0)
        assert got.down.data.tobytes() == spec.down.data.tobytes()
    with pytest.raises(InvalidData, match="pass the primary GGUF shard"):
        G.Gguf.open(paths[1])
    os.rename(paths[0], tmp_path / "renamed.gguf")
    with pytest.raises(InvalidData, match="invalid split filename"):
        G.Gguf.open(tmp_path / "renamed.gguf")
    os.rename(tmp_path / "renamed.gguf", paths[0])
    os.remove(paths[2])
    with pytest.raises(FileNotFoundError):
        G.Gguf.open(paths[0])


@pytest.mark.parametrize("fault", ["metadata", "split.no", "count", "duplicate"])
def test_split_model_inconsistencies(tmp_path, fault):
    spec, meta, tensors, paths = shard_model(tmp_path, 2)
    os.remove(paths[1])
    extra = {"general.architecture": "qwen4exp", "split.no": (G.T_U16, 1), "split.count": (G.T_U16, 2),
             "split.tensors.count": (G.T_I32, len(tensors))}
    second = list(tensors[1::2])
    if fault == "metadata":
        extra["qwen4exp.expert_count"] = 5
    elif fault == "split.no":
        extra["split.no"] = (G.T_U16, 0)
    elif fault == "count":
        second = second[:-1]
    else:
        second.append(tensors[0])
    G.write_gguf(paths[1], extra, second)
    with pytest.raises(InvalidData):
        G.Gguf.open(paths[0])


# -------------------------------------------------------- moe-layer command
def test_rust_debug_float_format():
    """Rust's {:?} of f32: shortest round-trip digits, '.0' on integers,
    exponent form below 1e-4 and from 1e16."""
    cases = {0.1: "0.1", 1.0: "1.0", 0.25: "0.25", 1 / 3: "0.33333334", 1e-4: "0.0001", 9.999e-5: "9.999e-5",
             1e-5: "1e-5", 1.5e-5: "1.5e-5", 1e16: "1e16", 123456789.0: "123456790.0", -0.0: "-0.0",
             3.4028235e38: "3.4028235e38", 1e-45: "1e-45", math.inf: "inf", math.nan: "NaN"}
    for v, s in cases.items():
        assert rust_f32(v) == s, v


def qwen_model(tmp_path):
    spec = CF.make_layer(53, 0, 512, 8, 2, 256, IQ2_XS, IQ2_XS, shared_ffn=256, shared_gate_kind=Q8_0,
                         shared_down_kind=Q8_0, shared_gated=True)
    p = str(tmp_path / "q.gguf")
    G.write_gguf(p, G.layer_metadata(spec, "qwen4exp", 1), G.layer_tensors(spec, 0))
    return spec, p


def run_cli(capsys, args):
    rc = main([str(a) for a in args])
    cap = capsys.readouterr()
    return rc, cap.out, cap.err


def test_moe_layer_argument_and_input_errors(tmp_path, capsys):
    """src/main.rs:255-293: every check before the GPU, each an 'ingot: ...'
    line on stderr, status 1, and no output file."""
    spec, model = qwen_model(tmp_path)
    good = tmp_path / "x.f32"
    CF.inputs(53, 1, 512)[0].astype("<f4").tofile(good)
    out = tmp_path / "out.f32"
    other = str(tmp_path / "other.gguf")
    G.write_gguf(other, {"general.architecture": "llama"}, [])
    short = tmp_path / "short.f32"
    np.zeros(511, "<f4").tofile(short)
    nan = tmp_path / "nan.f32"
    np.full(512, np.nan, "<f4").tofile(nan)
    inf = tmp_path / "inf.f32"
    v = np.zeros(512, "<f4")
    v[7] = np.inf
    v.tofile(inf)
    cases = [
        ([model, 0, good], USAGE),
        ([model, 0, good, out, "extra"], USAGE),
        ([model, "x", good, out], "invalid digit"),
        ([model, "-1", good, out], "invalid digit"),
        ([model, "", good, out], "empty string"),
        ([tmp_path / "missing.gguf", 0, good, out], "No such file"),
        ([other, 0, good, out], "only qwen4exp is supported"),
        ([model, 1, good, out], "layer out of range"),
        ([model, 0, tmp_path / "missing.f32", out], "No such file"),
        ([model, 0, short, out], "expected 512 little-endian F32 input values"),
        ([model, 0, nan, out], "input contains non-finite values"),
        ([model, 0, inf, out], "input contains non-finite values"),
    ]
    for args, msg in cases:
        rc, so, se = run_cli(capsys, args)
        assert rc == 1 and so == "" and se.startswith("ingot: ") and msg in se, (args, se)
        assert not out.exists()


def test_moe_layer_missing_tensors_and_keys(tmp_path, capsys):
    spec, _ = qwen_model(tmp_path)
    x = tmp_path / "x.f32"
    CF.inputs(53, 1, 512)[0].astype("<f4").tofile(x)
    meta = G.layer_metadata(spec, "qwen4exp", 1)
    del meta["qwen4exp.expert_shared_feed_forward_length"]
    p = str(tmp_path / "nokey.gguf")
    G.write_gguf(p, meta, G.layer_tensors(spec, 0))
    rc, _, se = run_cli(capsys, [p, 0, x, tmp_path / "o.f32"])
    assert rc == 1 and "missing integer: qwen4exp.expert_shared_feed_forward_length" in se
    p2 = str(tmp_path / "norouter.gguf")
    G.write_gguf(p2, G.layer_metadata(spec, "qwen4exp", 1), G.layer_tensors(spec, 0)[1:])
    rc, _, se = run_cli(capsys, [p2, 0, x, tmp_path / "o.f32"])
    assert rc == 1 and "missing tensor: blk.0.ffn_gate_inp.weight" in se
    assert not (tmp_path / "o.f32").exists()


@pytest.mark.parametrize("kind", [1, 30, 8])
def test_layer_spec_16_bit_router(tmp_path, kind):
    """F16 and BF16 routers and gate vectors widen exactly to float32; other
    types are refused for these small tensors."""
    spec = CF.make_layer(54, 0, 256, 4, 2, 256, Q8_0, Q8_0, shared_ffn=256, shared_gated=True)
    tensors = []
    for name, dims, k, data in G.layer_tensors(spec, 0):
        if "gate_inp" in name:
            v = np.frombuffer(np.ascontiguousarray(data).tobytes(), "<f4")
            if kind == 1:
                data = v.astype("<f2")
            elif kind == 30:
                data = (CF.round_bf16(v).view(np.uint32) >> 16).astype("<u2")
            else:
                data = CF.quantize(Q8_0, v.reshape(1, -1)).data
            k = kind
        tensors.append((name, dims, k, data))
    p = str(tmp_path / "r.gguf")
    G.write_gguf(p, G.layer_metadata(spec, "qwen4exp", 1), tensors)
    with G.Gguf.open(p) as g:
        if kind == 8:
            with pytest.raises(InvalidData, match="expected F32, F16 or BF16"):
                G.layer_spec(g, 0)
            return
        got = G.layer_spec(g, 0)
        widen = (lambda v: v.astype(np.float16).astype(np.float32)) if kind == 1 else CF.round_bf16
        assert got.router.dtype == np.float32 and np.array_equal(got.router, widen(spec.router))
        assert np.array_equal(got.shared_gate_vec, widen(spec.shared_gate_vec))
