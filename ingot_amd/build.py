"""Builds the native libraries in-tree (no JIT cache: the .so files travel with the tree).

    python -m ingot_amd.build            # HIP backend + synth library + CPU oracle

* ingot_amd/libingot_moe.so   hipcc --offload-arch=gfx950 (kernels + C ABI; the
                              csrc/*.hip units compiled in parallel, then linked)
* ingot_amd/libingot_synth.so g++ (synthetic inputs, quantizers)
* oracle/liboracle.so         make -C oracle (CPU oracle, test infrastructure)
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

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


def hip_sources() -> list[str]:
    """moe_hip.hip (C ABI, format-independent kernels) and the kinds_*.hip
    units, each of which instantiates the kernels of a few GGUF formats."""
    kinds = sorted(f for f in os.listdir(CSRC) if f.startswith("kinds_") and f.endswith(".hip"))
    return [os.path.join(CSRC, "moe_hip.hip")] + [os.path.join(CSRC, f) for f in kinds]


def build_hip(verbose: bool = False, jobs: int = 0) -> str:
    """Compiles every unit to an object in parallel, then links libingot_moe.so."""
    out = os.path.join(HERE, "libingot_moe.so")
    srcs = hip_sources()
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", "0")) or os.cpu_count() or 1)
    flags = [f for f in HIP_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="ingot_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(f)[:-4] + ".o") for f in srcs]
        cmds = [[HIPCC, *flags, "-c", "-o", o, f] for f, o in zip(srcs, objs)]
        with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", _atomic(out), *objs], verbose)
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
