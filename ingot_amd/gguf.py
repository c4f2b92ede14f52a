"""Validated GGUF v3 directories, expert slabs and resident layers.

Mirrors the reference's reader (src/gguf.rs) for the MoE path:

* ``Gguf.open``      directory parse and checks (src/gguf.rs:117-203) and split
                     shards ``NAME-0000k-of-0000n.gguf`` (:205-271)
* metadata           ``integer`` / ``float`` / ``string`` / ``array`` /
                     ``integers`` / ``strings`` and their optional forms
                     (:272-326); integers of every width read as unsigned,
                     F32/F64 as float (:87-116)
* ``tensor``         dims, type, absolute offset, shard, row stride and bytes
                     (:18-25, :327-331)
* ``read_range`` /
  ``rows`` /
  ``matrix``         positional reads of a range, of rows and of expert slabs
                     of a ``[cols, rows, E]`` tensor (:346-351, :404-460)
* ``map_tensor``     the tensor's bytes as a read-only memory map (:352-375)
* ``ffn_weights``    gate, up and down slabs of selected experts or of the
                     shared expert (src/lib.rs:62-88)
* ``geometry``       (values per block, bytes per block) per GGML type
                     (src/gguf.rs:470-491)

Errors are ``InvalidData`` (src/lib.rs:39-41), except a file truncated after
its directory was validated, which raises ``EOFError`` (the reference's
io::ErrorKind::UnexpectedEof). ``layer_spec`` assembles a resident
``LayerSpec`` for one layer (router, every expert, shared expert and its
gate) from memory maps, so the weights go from the page cache to HBM once,
in ``MoeLayer``. ``write_gguf`` writes the same format from raw block bytes;
tests use it for fixtures.
"""
from __future__ import annotations

import os
import struct
import time
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from .moe import InvalidData, LayerSpec, Matrix, ROUTE_SIGMOID, ROUTE_SOFTMAX
from .moe import geometry as _geometry

MAGIC = 0x46554747  # "GGUF", little-endian
VERSION = 3

# Metadata value types.
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64, T_I64, T_F64 = range(13)


def geometry(kind: int) -> tuple[int, int]:
    """(values per block, bytes per block) of a GGML type (src/gguf.rs:470-491);
    InvalidData for a type the table does not name."""
    return _geometry(kind)


@dataclass
class Tensor:
    """src/gguf.rs:18-25: absolute `offset` in shard `shard`."""

    dims: list
    kind: int
    offset: int
    shard: int
    stride: int
    bytes: int


class _Reader:
    def __init__(self, f, size: int):
        self.f, self.size = f, size

    def bytes(self, n: int) -> bytes:
        if n > self.size - self.f.tell():
            raise InvalidData("truncated GGUF value")
        return self.f.read(n)

    def u32(self) -> int:
        return struct.unpack("<I", self.bytes(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.bytes(8))[0]

    def string(self) -> str:
        n = self.u64()
        try:
            return self.bytes(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise InvalidData(str(e)) from None

    def value(self, kind: int):
        # Integers (of any width and signedness, and bools) read as unsigned,
        # floats as float, as the reference's Value (src/gguf.rs:10-16, :86-115).
        if kind == T_STRING:
            return self.string()
        if kind == T_ARRAY:
            element = self.u32()
            if element == T_ARRAY:
                raise InvalidData("nested GGUF arrays")
            n = self.u64()
            if n > self.size - self.f.tell():
                raise InvalidData("truncated GGUF array")
            return [self.value(element) for _ in range(n)]
        if kind in (T_U8, T_I8, T_BOOL):
            return self.bytes(1)[0]
        if kind in (T_U16, T_I16):
            return struct.unpack("<H", self.bytes(2))[0]
        if kind in (T_U32, T_I32):
            return self.u32()
        if kind in (T_U64, T_I64):
            return self.u64()
        if kind == T_F32:
            return float(struct.unpack("<f", self.bytes(4))[0])
        if kind == T_F64:
            return float(struct.unpack("<d", self.bytes(8))[0])
        raise InvalidData(f"unknown GGUF metadata type {kind}")

    def directory(self, shard: int) -> tuple[dict, dict]:
        if self.u32() != MAGIC or self.u32() != VERSION:
            raise InvalidData("expected little-endian GGUF v3")
        nt, nm = self.u64(), self.u64()
        metadata = {}
        for _ in range(nm):
            key = self.string()
            kind = self.u32()
            value = self.value(kind)
            if key in metadata:
                raise InvalidData("duplicate GGUF metadata")
            metadata[key] = value
        alignment = metadata.get("general.alignment", 32)
        if isinstance(alignment, (float, str, list)):
            raise InvalidData("invalid alignment metadata")
        if alignment <= 0 or alignment & (alignment - 1):
            raise InvalidData("invalid GGUF alignment")
        tensors = {}
        for _ in range(nt):
            name = self.string()
            rank = self.u32()
            if not 1 <= rank <= 4:
                raise InvalidData("invalid tensor rank")
            dims = [self.u64() for _ in range(rank)]
            kind = self.u32()
            offset = self.u64()
            block, size = geometry(kind)
            if 0 in dims or dims[0] % block != 0 or offset % alignment != 0:
                raise InvalidData(f"invalid shape/alignment for {name}")
            stride = dims[0] // block * size
            nbytes = stride
            for d in dims[1:]:
                nbytes *= d
            if name in tensors:
                raise InvalidData("duplicate tensor")
            tensors[name] = Tensor(dims, kind, offset, shard, stride, nbytes)
        start = (self.f.tell() + alignment - 1) & ~(alignment - 1)
        ranges = []
        for name, t in tensors.items():
            t.offset += start
            end = t.offset + t.bytes
            if end > self.size:
                raise InvalidData(f"{name}: extends beyond file")
            ranges.append((t.offset, end))
        ranges.sort()
        if any(a[1] > b[0] for a, b in zip(ranges, ranges[1:])):
            raise InvalidData("overlapping tensor ranges")
        return tensors, metadata


def _directory(path: str, shard: int) -> tuple[dict, dict]:
    with open(path, "rb") as f:
        return _Reader(f, os.fstat(f.fileno()).st_size).directory(shard)


def _same(a, b) -> bool:
    """Value equality with the reference's variants kept apart (an integer
    never equals a float; src/gguf.rs:10-16 derives PartialEq)."""
    if type(a) is not type(b):
        return False
    if isinstance(a, list):
        return len(a) == len(b) and all(_same(x, y) for x, y in zip(a, b))
    return a == b


class Gguf:
    """A validated GGUF v3 model, possibly split in shards (src/gguf.rs:44-52).

    The shard files stay open until ``close``; reads are positional."""

    def __init__(self, files: list, tensors: dict, metadata: dict):
        self.files = files
        self.tensors = tensors
        self.metadata = metadata
        self.bytes_read = 0
        self.row_read_time = 0.0
        arch = metadata.get("general.architecture")
        if not isinstance(arch, str):
            raise InvalidData("missing architecture")
        self.architecture = arch

    def close(self) -> None:
        for f in self.files:
            f.close()
        self.files = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @classmethod
    def open(cls, path) -> "Gguf":
        """src/gguf.rs:204-258: the primary shard and, for split.count > 1,
        NAME-0000k-of-0000n.gguf beside it, each validated and consistent."""
        path = os.fspath(path)
        tensors, metadata = _directory(path, 0)
        g = cls([open(path, "rb")], tensors, metadata)
        try:
            count = g.optional_integer("split.count") or 1
            if count > 1:
                if g.integer("split.no") != 0:
                    raise InvalidData("pass the primary GGUF shard")
                base = os.path.basename(path)
                marker = f"-00001-of-{count:05d}.gguf"
                if not base.endswith(marker):
                    raise InvalidData("invalid split filename")
                prefix = base[: -len(marker)]
                for shard in range(1, count):
                    nxt = os.path.join(os.path.dirname(path), f"{prefix}-{shard + 1:05d}-of-{count:05d}.gguf")
                    f = open(nxt, "rb")
                    g.files.append(f)
                    t, m = _Reader(f, os.fstat(f.fileno()).st_size).directory(shard)
                    if (not _same(m.get("split.no"), shard) or not _same(m.get("split.count"), count)
                            or not _same(m.get("split.tensors.count"), metadata.get("split.tensors.count"))):
                        raise InvalidData("inconsistent GGUF shards")
                    for k, v in m.items():
                        if not k.startswith("split.") and k in metadata and not _same(metadata[k], v):
                            raise InvalidData(f"inconsistent shard metadata: {k}")
                    for name, tt in t.items():
                        if name in g.tensors:
                            raise InvalidData("duplicate tensor across shards")
                        g.tensors[name] = tt
                if g.integer("split.tensors.count") != len(g.tensors):
                    raise InvalidData("split tensor count mismatch")
        except BaseException:
            g.close()
            raise
        return g

    # -------------------------------------------------------------- metadata
    def optional_integer(self, key: str) -> Optional[int]:
        v = self.metadata.get(key)
        return v if isinstance(v, int) else None

    def integer(self, key: str) -> int:
        v = self.optional_integer(key)
        if v is None:
            raise InvalidData(f"missing integer: {key}")
        return v

    def float(self, key: str) -> float:
        """An F32/F64 value narrowed to f32, which must be finite."""
        v = self.metadata.get(key)
        if isinstance(v, float):
            with np.errstate(over="ignore"):
                f = np.float32(v)
            if np.isfinite(f):
                return float(f)
        raise InvalidData(f"missing float: {key}")

    def optional_float(self, key: str) -> Optional[float]:
        try:
            return self.float(key)
        except InvalidData:
            return None

    def optional_string(self, key: str) -> Optional[str]:
        v = self.metadata.get(key)
        return v if isinstance(v, str) else None

    def string(self, key: str) -> str:
        v = self.optional_string(key)
        if v is None:
            raise InvalidData(f"missing string: {key}")
        return v

    def array(self, key: str) -> list:
        v = self.metadata.get(key)
        if not isinstance(v, list):
            raise InvalidData(f"missing array: {key}")
        return v

    def integers(self, key: str) -> list:
        a = self.array(key)
        if not all(isinstance(v, int) for v in a):
            raise InvalidData(key)
        return list(a)

    def strings(self, key: str) -> list:
        a = self.array(key)
        if not all(isinstance(v, str) for v in a):
            raise InvalidData(key)
        return list(a)

    # ---------------------------------------------------------------- tensors
    def tensor(self, name: str) -> Tensor:
        t = self.tensors.get(name)
        if t is None:
            raise InvalidData(f"missing tensor: {name}")
        return t

    def _location(self, t: Tensor, offset: int, length: int):
        if offset < 0 or length < 0 or offset + length > t.bytes:
            raise InvalidData("tensor read out of bounds")
        if not 0 <= t.shard < len(self.files):
            raise InvalidData("invalid tensor shard")
        return self.files[t.shard], t.offset + offset

    def read_range(self, t: Tensor, offset: int, length: int) -> bytes:
        """`length` bytes at `offset` into tensor `t` (src/gguf.rs:346-351);
        EOFError when the file has been truncated since it was opened."""
        f, start = self._location(t, offset, length)
        data = os.pread(f.fileno(), length, start)
        if len(data) != length:
            raise EOFError("failed to fill whole buffer")
        self.bytes_read += length
        return data

    def map_tensor(self, t: Tensor) -> np.ndarray:
        """The tensor's bytes as a read-only memory map (src/gguf.rs:352-374).
        The file must stay unchanged while the mapping lives."""
        f, start = self._location(t, 0, t.bytes)
        if start + t.bytes > os.fstat(f.fileno()).st_size:
            raise EOFError("mapped tensor was truncated")
        return np.memmap(f, dtype=np.uint8, mode="r", offset=start, shape=(t.bytes,))

    def rows(self, name: str, rows: Sequence[int]) -> Matrix:
        """Rows `rows` of a tensor in that order, repeats allowed
        (src/gguf.rs:401-433). Every row is read before a failure is
        raised; the rows that were read count in `bytes_read`."""
        t = self.tensor(name)
        n = t.bytes // t.stride
        if len(rows) == 0 or any(r < 0 or r >= n for r in rows):
            raise InvalidData("row out of range")
        started = time.perf_counter()
        parts, error = [], None
        for r in rows:
            try:
                parts.append(self.read_range(t, int(r) * t.stride, t.stride))
            except (OSError, EOFError) as e:
                error = error or e
        self.row_read_time += time.perf_counter() - started
        if error is not None:
            raise error
        return Matrix(np.frombuffer(b"".join(parts), np.uint8).copy(), t.dims[0], len(rows), 1, t.kind, t.stride)

    def matrix(self, name: str, shape: Sequence[int], experts: Sequence[int], copy: bool = True) -> Matrix:
        """Expert slabs `experts` of a tensor whose dims equal `shape`
        ([cols, rows, E], [cols, rows] or [cols]) (src/gguf.rs:434-460).
        copy=False maps the file instead of reading it when `experts` is one
        ascending run (resident layers)."""
        t = self.tensor(name)
        if list(t.dims) != list(shape):
            raise InvalidData(f"{name}: expected {list(shape)}, found {list(t.dims)}")
        rows = shape[1] if len(shape) > 1 else 1
        count = shape[2] if len(shape) > 2 else 1
        ex = [int(e) for e in experts]
        if len(ex) == 0 or any(e < 0 or e >= count for e in ex):
            raise InvalidData("expert out of range")
        size = t.stride * rows
        if not copy and ex == list(range(ex[0], ex[0] + len(ex))):
            data = self.map_tensor(t)[ex[0] * size:(ex[0] + len(ex)) * size]
        else:
            data = np.frombuffer(b"".join(self.read_range(t, e * size, size) for e in ex), np.uint8).copy()
        return Matrix(data, shape[0], rows, len(ex), t.kind, t.stride)


def ffn_weights(model: Gguf, layer: int, width: int, hidden: int, count: int, ids: Sequence[int],
                shared: bool) -> tuple[Matrix, Matrix, Matrix]:
    """src/lib.rs:62-88: blk.L.ffn_{gate,up,down}_{exps|shexp}.weight slabs."""
    suffix = "shexp" if shared else "exps"

    def load(name, cols, rows):
        shape = [cols, rows] if shared else [cols, rows, count]
        return model.matrix(f"blk.{layer}.ffn_{name}_{suffix}.weight", shape, ids)

    return load("gate", width, hidden), load("up", width, hidden), load("down", hidden, width)


def _f32_tensor(model: Gguf, name: str, shape: Sequence[int]) -> np.ndarray:
    """A small F32, F16 or BF16 tensor (router, bias, gate vector, norm gain)
    as float32. The two 16-bit types widen exactly (the same values the GPU's
    project path decodes); any other type is refused, as Weight::require_f32
    (src/glm.rs:425) refuses non-F32 norms."""
    m = model.matrix(name, shape, [0])
    raw = np.ascontiguousarray(m.data)
    if m.kind == 0:
        return raw.view("<f4").astype(np.float32)
    if m.kind == 1:
        return raw.view("<f2").astype(np.float32)
    if m.kind == 30:
        return (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
    raise InvalidData(f"{name}: expected F32, F16 or BF16")


def layer_spec(model: Gguf, layer: int, norm: bool = False) -> LayerSpec:
    """A resident LayerSpec for MoE layer `layer` of `model`.

    Keys carry the architecture prefix: {arch}.block_count,
    .embedding_length, .expert_count, .expert_used_count,
    .expert_feed_forward_length and, for a shared expert,
    .expert_shared_feed_forward_length (src/main.rs:269-279, src/qwen.rs:163).
    Tensors: blk.L.ffn_gate_inp.weight [H, E] (F32), the three
    ffn_*_exps slabs [.., .., E] mapped whole (no copy), the shared
    ffn_*_shexp matrices and the ffn_gate_inp_shexp.weight [H] gate when
    present (src/qwen.rs:499-504). {arch}.expert_gating_func == 2 selects
    sigmoid routing with {arch}.expert_weights_scale and the
    blk.L.exp_probs_b.bias correction bias (src/glm.rs:72, :99, :424).
    norm=True adds the blk.L.ffn_norm.weight gain and
    {arch}.attention.layer_norm_rms_epsilon, so the layer computes
    x + MoE(RMSNorm(x)); the default computes MoE(x), the FFN input the
    reference's moe-layer harness takes."""
    a = model.architecture
    if layer < 0 or layer >= model.integer(f"{a}.block_count"):
        raise InvalidData("layer out of range")
    width = model.integer(f"{a}.embedding_length")
    count = model.integer(f"{a}.expert_count")
    top = model.integer(f"{a}.expert_used_count")
    hidden = model.integer(f"{a}.expert_feed_forward_length")
    p = f"blk.{layer}."
    router = _f32_tensor(model, p + "ffn_gate_inp.weight", [width, count]).reshape(count, width)
    gate, up, down = (model.matrix(f"{p}ffn_{n}_exps.weight", s, range(count), copy=False)
                      for n, s in (("gate", [width, hidden, count]), ("up", [width, hidden, count]),
                                   ("down", [hidden, width, count])))
    spec = LayerSpec(hidden=width, experts=count, top_k=top, router=router, gate=gate, up=up, down=down)
    if model.optional_integer(f"{a}.expert_gating_func") == 2:
        spec.routing = ROUTE_SIGMOID
        spec.route_scale = model.optional_float(f"{a}.expert_weights_scale") or 1.0
        if p + "exp_probs_b.bias" in model.tensors:
            spec.router_bias = _f32_tensor(model, p + "exp_probs_b.bias", [count])
    if p + "ffn_gate_shexp.weight" in model.tensors:
        sh = model.optional_integer(f"{a}.expert_shared_feed_forward_length") or hidden
        spec.shared = tuple(model.matrix(f"{p}ffn_{n}_shexp.weight", s, [0], copy=False)
                            for n, s in (("gate", [width, sh]), ("up", [width, sh]), ("down", [sh, width])))
        if p + "ffn_gate_inp_shexp.weight" in model.tensors:
            spec.shared_gate_vec = _f32_tensor(model, p + "ffn_gate_inp_shexp.weight", [width])
    if norm:
        spec.norm_gain = _f32_tensor(model, p + "ffn_norm.weight", [width])
        spec.norm_eps = model.float(f"{a}.attention.layer_norm_rms_epsilon")
    return spec


# ------------------------------------------------------------------ writer
def _value(kind: int, v) -> bytes:
    if kind == T_STRING:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if kind == T_ARRAY:
        ek, items = v
        return struct.pack("<IQ", ek, len(items)) + b"".join(_value(ek, x) for x in items)
    fmt = {T_U8: "<B", T_I8: "<b", T_BOOL: "<B", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
           T_U64: "<Q", T_I64: "<q", T_F32: "<f", T_F64: "<d"}[kind]
    return struct.pack(fmt, v)


def _infer(v) -> tuple[int, object]:
    if isinstance(v, bool):
        return T_BOOL, int(v)
    if isinstance(v, int):
        return (T_U32, v) if 0 <= v < 2 ** 32 else (T_U64, v)
    if isinstance(v, float):
        return T_F32, v
    if isinstance(v, str):
        return T_STRING, v
    if isinstance(v, (list, tuple)):
        k = _infer(v[0])[0] if v else T_U32
        return T_ARRAY, (k, [_infer(x)[1] for x in v])
    raise TypeError(f"cannot write metadata value {v!r}")


def write_gguf(path: str, metadata: dict, tensors: Sequence[tuple], alignment: int = 32) -> None:
    """Writes a GGUF v3 file. `metadata`: key -> value (int, float, str, bool,
    list) or (type, value); `tensors`: (name, dims, kind, bytes) with the
    tensor's raw block bytes. An alignment other than 32 is recorded as
    general.alignment. Refuses to replace an existing file."""
    if alignment != 32:
        metadata = {**metadata, "general.alignment": (T_U32, alignment)}
    header = bytearray(struct.pack("<IIQQ", MAGIC, VERSION, len(tensors), len(metadata)))
    for key, v in metadata.items():
        kind, val = v if isinstance(v, tuple) and len(v) == 2 and isinstance(v[0], int) else _infer(v)
        header += _value(T_STRING, key) + struct.pack("<I", kind) + _value(kind, val)
    offset, blobs = 0, []
    for name, dims, kind, data in tensors:
        data = np.ascontiguousarray(data).tobytes() if isinstance(data, np.ndarray) else bytes(data)
        header += _value(T_STRING, name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        header += struct.pack("<IQ", kind, offset)
        blobs.append((offset, data))
        offset += (len(data) + alignment - 1) // alignment * alignment
    header += b"\0" * ((-len(header)) % alignment)
    with open(path, "xb") as f:
        f.write(header)
        for off, data in blobs:
            f.write(data)
            f.write(b"\0" * ((-len(data)) % alignment))


def write_split(path_prefix: str, metadata: dict, tensors: Sequence[tuple], shards: int,
                alignment: int = 32) -> list:
    """Writes `tensors` over `shards` files PREFIX-0000k-of-0000n.gguf (tensors
    dealt round-robin, the full metadata in the first shard, the split keys in
    every shard) and returns their paths, the first one first."""
    paths = [f"{path_prefix}-{k + 1:05d}-of-{shards:05d}.gguf" for k in range(shards)]
    for k, path in enumerate(paths):
        meta = dict(metadata) if k == 0 else {"general.architecture": metadata["general.architecture"]}
        meta.update({"split.no": (T_U16, k), "split.count": (T_U16, shards),
                     "split.tensors.count": (T_I32, len(tensors))})
        write_gguf(path, meta, list(tensors[k::shards]), alignment)
    return paths


def layer_tensors(spec: LayerSpec, layer: int) -> list:
    """The (name, dims, kind, bytes) tensors of one MoE layer in GGUF naming,
    the inverse of `layer_spec`."""
    p = f"blk.{layer}."
    f32 = lambda a: np.ascontiguousarray(a, dtype="<f4").view(np.uint8).ravel()  # noqa: E731
    out = [(p + "ffn_gate_inp.weight", [spec.hidden, spec.experts], 0, f32(spec.router))]
    for n, m in (("gate", spec.gate), ("up", spec.up), ("down", spec.down)):
        out.append((f"{p}ffn_{n}_exps.weight", [m.cols, m.rows, m.count], m.kind, m.data))
    if spec.router_bias is not None:
        out.append((p + "exp_probs_b.bias", [spec.experts], 0, f32(spec.router_bias)))
    if spec.shared is not None:
        for n, m in zip(("gate", "up", "down"), spec.shared):
            out.append((f"{p}ffn_{n}_shexp.weight", [m.cols, m.rows], m.kind, m.data))
    if spec.shared_gate_vec is not None:
        out.append((p + "ffn_gate_inp_shexp.weight", [spec.hidden], 0, f32(spec.shared_gate_vec)))
    if spec.norm_gain is not None:
        out.append((p + "ffn_norm.weight", [spec.hidden], 0, f32(spec.norm_gain)))
    return out


def layer_metadata(spec: LayerSpec, arch: str, blocks: int) -> dict:
    """The {arch}.* keys `layer_spec` reads for `spec`."""
    m = {"general.architecture": arch, f"{arch}.block_count": blocks, f"{arch}.embedding_length": spec.hidden,
         f"{arch}.expert_count": spec.experts, f"{arch}.expert_used_count": spec.top_k,
         f"{arch}.expert_feed_forward_length": spec.gate.rows}
    if spec.shared is not None:
        m[f"{arch}.expert_shared_feed_forward_length"] = spec.shared[0].rows
    if spec.routing == ROUTE_SIGMOID:
        m[f"{arch}.expert_gating_func"] = 2
        m[f"{arch}.expert_weights_scale"] = float(spec.route_scale)
    if spec.norm_gain is not None:
        m[f"{arch}.attention.layer_norm_rms_epsilon"] = float(spec.norm_eps)
    return m

