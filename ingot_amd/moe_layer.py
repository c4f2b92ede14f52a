"""One MoE FFN of a real qwen4exp GGUF on the GPU.

    python -m ingot_amd.moe_layer MODEL.gguf LAYER INPUT.f32 OUTPUT.f32

The reference's ``ingot dev moe-layer`` (src/main.rs:255-325), with the same
checks, in the same order, and the same output:

* exactly four arguments; LAYER a non-negative decimal integer;
* the model opens as validated GGUF v3 (a split model through its first
  shard) with general.architecture ``qwen4exp`` and LAYER below
  qwen4exp.block_count;
* INPUT holds exactly qwen4exp.embedding_length little-endian F32 values,
  all finite;
* router logits ``blk.L.ffn_gate_inp.weight [H, E]`` · x on the GPU, top-K
  routing (ties to the lower id), the K selected routed experts and the
  shared expert read from the file (src/lib.rs:62-88), and the shared
  expert's sigmoid gate ``blk.L.ffn_gate_inp_shexp.weight [H]``;
* OUTPUT is created only after the layer succeeded and never replaces an
  existing file;
* stdout: ``device=``, ``selected_experts=``, ``routing_weights=`` (as Rust
  prints a Vec<f32>) and ``output_values=``.

Errors print ``ingot: <message>`` on stderr and exit with status 1
(src/main.rs:327-335). The check that feeds the same files to this command
and compares against a ggml dequantization (tools/check_rust_moe.py) parses
exactly these lines.
"""
from __future__ import annotations

import os
import re
import sys
from typing import Optional, Sequence

import numpy as np

from .gguf import Gguf, ffn_weights
from .moe import Gpu, InvalidData

USAGE = "usage: ingot dev moe-layer MODEL.gguf LAYER INPUT.f32 OUTPUT.f32"


def rust_f32(v) -> str:
    """A float32 as Rust's `{:?}` writes it: the shortest digits that read
    back to the same f32, a decimal point always, exponent form below 1e-4
    and from 1e16."""
    f = np.float32(v)
    if not np.isfinite(f):
        return "NaN" if np.isnan(f) else ("inf" if f > 0 else "-inf")
    a = np.abs(f)  # compared as f32, like the f32 literals in Rust's rule
    if a != 0 and (a < np.float32(1e-4) or a >= np.float32(1e16)):
        mant, exp = np.format_float_scientific(f, unique=True, trim="-").split("e")
        return f"{mant}e{int(exp)}"
    return np.format_float_positional(f, unique=True, trim="0")


def _layer_index(text: str) -> int:
    # usize::from_str: an optional '+' and decimal digits only.
    if not re.fullmatch(r"\+?[0-9]+", text):
        raise InvalidData("cannot parse integer from empty string" if text == "" else "invalid digit found in string")
    return int(text)


def moe_layer(args: Sequence[str], gpu: Optional[Gpu] = None) -> str:
    """args: [MODEL, LAYER, INPUT, OUTPUT]. Returns the report printed on
    stdout; raises InvalidData / OSError as the reference returns them."""
    if len(args) != 4:
        raise InvalidData(USAGE)
    layer = _layer_index(args[1])
    with Gguf.open(args[0]) as model:
        if model.architecture != "qwen4exp":
            raise InvalidData("only qwen4exp is supported")
        if layer >= model.integer("qwen4exp.block_count"):
            raise InvalidData("layer out of range")
        width = model.integer("qwen4exp.embedding_length")
        count = model.integer("qwen4exp.expert_count")
        top = model.integer("qwen4exp.expert_used_count")
        hidden = model.integer("qwen4exp.expert_feed_forward_length")
        shared_hidden = model.integer("qwen4exp.expert_shared_feed_forward_length")
        with open(args[2], "rb") as f:
            raw = f.read()
        if len(raw) != width * 4:
            raise InvalidData(f"expected {width} little-endian F32 input values")
        x = np.frombuffer(raw, dtype="<f4").astype(np.float32)
        if not np.isfinite(x).all():
            raise InvalidData("input contains non-finite values")
        router = model.matrix(f"blk.{layer}.ffn_gate_inp.weight", [width, count], [0])
        own = gpu is None
        if own:
            gpu = Gpu(0)
        try:
            ids, weights = gpu.route(gpu.project(router, x), top)
            routed = ffn_weights(model, layer, width, hidden, count, ids, False)
            shared = ffn_weights(model, layer, width, shared_hidden, 1, [0], True)
            shared_gate = model.matrix(f"blk.{layer}.ffn_gate_inp_shexp.weight", [width], [0])
            out = gpu.moe(routed, shared, shared_gate, x, weights)
            name = gpu.name()
        finally:
            if own:
                gpu.close()
    # Do not replace an existing artifact, model or input by accident.
    with open(args[3], "xb") as f:
        f.write(np.asarray(out, dtype="<f4").tobytes())
    return (f"device={name}\n"
            f"selected_experts=[{', '.join(str(i) for i in ids)}]\n"
            f"routing_weights=[{', '.join(rust_f32(w) for w in weights)}]\n"
            f"output_values={width}")


def main(argv: Optional[Sequence[str]] = None) -> int:
    try:
        print(moe_layer(list(sys.argv[1:] if argv is None else argv)), flush=True)
        return 0
    except (InvalidData, OSError, EOFError, RuntimeError) as e:
        msg = e.strerror if isinstance(e, OSError) and e.strerror else str(e)
        if isinstance(e, OSError) and e.filename:
            msg = f"{msg}: {os.fsdecode(e.filename)}"
        print(f"ingot: {msg}", file=sys.stderr, flush=True)
        return 1


if __name__ == "__main__":
    sys.exit(main())
