"""Builds the native libraries in-tree (no JIT cache: the .so files travel with the tree).

    python -m ingot_amd.build            # HIP backend + synth library + CPU oracle

* ingot_amd/libingot_moe.so   hipcc --offload-arch=gfx950 (kernels + C ABI)
* ingot_amd/libingot_synth.so g++ (synthetic inputs, quantizers)
* oracle/liboracle.so         make -C oracle (CPU oracle, test infrastructure)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("INGOT_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: never emit packed fp32 VALU instructions on gfx950.
HIP_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", "-mavx2", "-mfma", "-ffp-contract=off", "-pthread"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        lines = [l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l]
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n" + "\n".join(lines[-80:]))


def _atomic(out: str) -> str:
    return out + ".tmp"


def build_synth(verbose: bool = False) -> str:
    out = os.path.join(HERE, "libingot_synth.so")
    _run(["g++", *HOST_FLAGS, "-o", _atomic(out), os.path.join(CSRC, "synth.cpp")], verbose)
    os.replace(_atomic(out), out)
    return out


def build_hip(verbose: bool = False) -> str:
    out = os.path.join(HERE, "libingot_moe.so")
    _run([HIPCC, *HIP_FLAGS, "-o", _atomic(out), os.path.join(CSRC, "moe_hip.hip")], verbose)
    os.replace(_atomic(out), out)
    return out


def build_oracle(verbose: bool = False) -> str:
    _run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle")], verbose)
    return os.path.join(ROOT, "oracle", "liboracle.so")


def build_all(verbose: bool = False) -> None:
    build_synth(verbose)
    build_oracle(verbose)
    build_hip(verbose)


if __name__ == "__main__":
    build_all(verbose="-q" not in sys.argv)
