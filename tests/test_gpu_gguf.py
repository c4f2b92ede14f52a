"""GPU tests of GGUF models: the moe-layer command and resident layers read
from a file.

A synthetic two-layer qwen4exp model, split over two shards, stands in for
the real checkpoint (no model file travels here). The command is checked the
way the reference's own checker drives ``ingot dev moe-layer``
(tools/check_rust_moe.py:79-125): inputs "normal", "small" and "zero_ties";
expert ids exact, routing weights within rtol 2e-5 / atol 2e-7, outputs
within the parity bar of tests/util.py; an existing output is never replaced
and a non-finite input writes nothing.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from ingot_amd import configs as CF
from ingot_amd import gguf as G
from ingot_amd.moe import BF16, IQ2_S, IQ2_XS, IQ3_S, IQ4_NL, IQ4_XS, Q2_0, Q4_K, Q8_0, MoeLayer
from ingot_amd.moe_layer import moe_layer
from util import assert_close, check_layer

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
H = 1024


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    """Layer 0: IQ2_XS experts with a gated Q8_0 shared expert (C2's formats);
    layer 1: Q4_K gate/up, IQ4_NL down, gated Q4_K/Q8_0 shared expert."""
    specs = [
        CF.make_layer(60, 0, H, 32, 4, 256, IQ2_XS, IQ2_XS, shared_ffn=512, shared_gate_kind=Q8_0,
                      shared_down_kind=Q8_0, shared_gated=True),
        CF.make_layer(60, 1, H, 32, 4, 256, Q4_K, IQ4_NL, shared_ffn=512, shared_gate_kind=Q4_K,
                      shared_down_kind=Q8_0, shared_gated=True),
    ]
    meta = G.layer_metadata(specs[0], "qwen4exp", 2)
    tensors = G.layer_tensors(specs[0], 0) + G.layer_tensors(specs[1], 1)
    d = tmp_path_factory.mktemp("gguf")
    paths = G.write_split(str(d / "synthetic-qwen4exp"), meta, tensors, 2)
    return specs, paths[0], d


def cases():
    rng = np.random.default_rng(20261011)  # tools/check_rust_moe.py:88-91
    return [("normal", rng.normal(size=H).astype(np.float32)),
            ("small", (rng.normal(size=H) * 0.01).astype(np.float32)),
            ("zero_ties", np.zeros(H, np.float32))]


def parse(report: str) -> dict:
    return dict(line.split("=", 1) for line in report.splitlines())


@pytest.mark.parametrize("layer", [0, 1])
def test_moe_layer_command_matches_oracle(gpu, oracle, model, layer):
    specs, path, d = model
    spec = specs[layer]
    for name, x in cases():
        inp, out = d / f"in-{layer}-{name}.f32", d / f"out-{layer}-{name}.f32"
        x.astype("<f4").tofile(inp)
        print(f"moe-layer layer={layer} case={name}", flush=True)
        lines = parse(moe_layer([path, str(layer), str(inp), str(out)], gpu))
        st, ref, ids, w = oracle.moe_forward(spec, x[None], oracle.F64)
        assert st == 0
        got_ids = json.loads(lines["selected_experts"])
        got_w = np.array(json.loads(lines["routing_weights"]), np.float32)
        assert got_ids == [int(i) for i in ids[0]], name
        np.testing.assert_allclose(got_w, w[0], rtol=2e-5, atol=2e-7)
        assert lines["output_values"] == str(H) and lines["device"] == gpu.name()
        got = np.fromfile(out, dtype="<f4")
        assert got.shape == (H,)
        if name == "zero_ties":
            assert got_ids == list(range(4)) and not got.any()
        else:
            assert_close(got, ref[0], f"moe-layer {layer} {name}")


def test_moe_layer_command_process_contract(model):
    """As the reference's checker runs it: a child process, stdout parsed,
    a second run onto the same output refused with the file unchanged, and a
    NaN input refused with no output written (tools/check_rust_moe.py:96-119)."""
    specs, path, d = model
    x = cases()[0][1]
    inp, out = d / "proc-in.f32", d / "proc-out.f32"
    x.astype("<f4").tofile(inp)
    cmd = [sys.executable, "-m", "ingot_amd.moe_layer", path, "0", str(inp), str(out)]
    env = dict(os.environ, PYTHONPATH=ROOT)
    run = subprocess.run(cmd, text=True, capture_output=True, timeout=120, env=env, cwd=ROOT)
    assert run.returncode == 0, run.stderr
    lines = parse(run.stdout)
    assert set(lines) == {"device", "selected_experts", "routing_weights", "output_values"}
    before = out.read_bytes()
    again = subprocess.run(cmd, text=True, capture_output=True, timeout=120, env=env, cwd=ROOT)
    assert again.returncode == 1 and again.stderr.startswith("ingot: ") and out.read_bytes() == before
    bad, bad_out = d / "bad.f32", d / "bad-out.f32"
    np.full(H, np.nan, np.float32).tofile(bad)
    fail = subprocess.run(cmd[:-2] + [str(bad), str(bad_out)], text=True, capture_output=True, timeout=120,
                          env=env, cwd=ROOT)
    assert fail.returncode == 1 and not bad_out.exists()


@pytest.mark.parametrize("layer", [0, 1])
def test_resident_layer_from_gguf(gpu, oracle, model, layer):
    """layer_spec maps every expert of the file; the resident layer on the GPU
    matches the oracle on decode and prefill batches."""
    specs, path, _ = model
    with G.Gguf.open(path) as g:
        spec = G.layer_spec(g, layer)
        assert spec.gate.data.tobytes() == specs[layer].gate.data.tobytes()
        resident = MoeLayer(gpu, spec)
        for T in (1, 4, 64):
            print(f"resident layer={layer} T={T}", flush=True)
            check_layer(resident, spec, CF.inputs(60, T, H, seed=layer), oracle, f"GGUF layer {layer} T={T}")
        resident.destroy()


def to_bf16(v):
    """float32 -> (bf16 bytes, the float32 values they hold), round to nearest even."""
    r = CF.round_bf16(np.asarray(v, np.float32))
    return (r.view(np.uint32) >> 16).astype("<u2"), r


def test_qwen38_style_format_mix(gpu, oracle, tmp_path):
    """The format mix of the reference's real-file record (validation/rust-moe-layer-0.json:
    BF16, IQ2_S, IQ3_S, IQ4_NL, IQ4_XS, Q2_0): BF16 router and shared gate, IQ2_S gate/up,
    IQ3_S down, IQ4_XS shared gate/up, Q2_0 shared down; through the command and as a
    resident layer."""
    spec = CF.make_layer(61, 0, H, 64, 8, 256, IQ2_S, IQ3_S, shared_ffn=512, shared_gate_kind=IQ4_XS,
                         shared_down_kind=Q2_0, shared_gated=True)
    rb, spec.router = to_bf16(spec.router)
    gb, spec.shared_gate_vec = to_bf16(spec.shared_gate_vec)
    tensors = []
    for name, dims, kind, data in G.layer_tensors(spec, 0):
        if name.endswith("ffn_gate_inp.weight"):
            tensors.append((name, dims, BF16, rb))
        elif name.endswith("ffn_gate_inp_shexp.weight"):
            tensors.append((name, dims, BF16, gb))
        else:
            tensors.append((name, dims, kind, data))
    path = str(tmp_path / "mix.gguf")
    G.write_gguf(path, G.layer_metadata(spec, "qwen4exp", 1), tensors)
    for name, x in cases():
        inp, out = tmp_path / f"in-{name}.f32", tmp_path / f"out-{name}.f32"
        x.astype("<f4").tofile(inp)
        print(f"mix moe-layer case={name}", flush=True)
        lines = parse(moe_layer([path, "0", str(inp), str(out)], gpu))
        st, ref, ids, w = oracle.moe_forward(spec, x[None], oracle.F64)
        assert json.loads(lines["selected_experts"]) == [int(i) for i in ids[0]]
        np.testing.assert_allclose(np.array(json.loads(lines["routing_weights"]), np.float32), w[0],
                                   rtol=2e-5, atol=2e-7)
        got = np.fromfile(out, dtype="<f4")
        if name == "zero_ties":
            assert not got.any()
        else:
            assert_close(got, ref[0], f"mix moe-layer {name}")
    with G.Gguf.open(path) as g:
        file_spec = G.layer_spec(g, 0)
        assert np.array_equal(file_spec.router, spec.router)
        resident = MoeLayer(gpu, file_spec)
        for T in (1, 4, 40):
            print(f"mix resident T={T}", flush=True)
            check_layer(resident, file_spec, CF.inputs(61, T, H, seed=T), oracle, f"mix resident T={T}")
        resident.destroy()
