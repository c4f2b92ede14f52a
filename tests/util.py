"""Shared checks for the parity tests.

The parity bar: expert indices bit-exact (ties to
the lower index); hidden outputs within max-abs 1e-3 and relative L2 1e-4 of
the CPU layer with fp32 accumulation. Both the fp32 CPU layer and the fp64
oracle are checked.
"""
import numpy as np

MAX_ABS = 1e-3
REL_L2 = 1e-4


def parity_metrics(out, ref):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    maxabs = float(np.abs(out - ref).max()) if out.size else 0.0
    denom = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(out - ref) / denom) if denom > 0 else float(np.linalg.norm(out - ref))
    return maxabs, rel


def assert_close(out, ref, what=""):
    maxabs, rel = parity_metrics(out, ref)
    assert maxabs <= MAX_ABS and rel <= REL_L2, f"{what}: max-abs {maxabs:.3e} rel-L2 {rel:.3e}"
    return maxabs, rel


def check_layer(layer, spec, x, oracle, label=""):
    """Runs the GPU layer and both oracle precisions on x; asserts the parity bar."""
    out, ids, w = layer(x)
    st64, o64, ids64, w64 = oracle.moe_forward(spec, x, oracle.F64)
    st32, o32, ids32, w32 = oracle.moe_forward(spec, x, oracle.F32)
    assert st64 == 0 and st32 == 0
    assert np.array_equal(ids64, ids32)
    assert np.array_equal(ids, ids64), f"{label}: expert ids differ from the oracle"
    # Routing weights use the same fixed fp32 operation sequence on both sides.
    assert np.array_equal(w, w64), f"{label}: routing weights differ"
    m64 = assert_close(out, o64, f"{label} vs fp64 oracle")
    m32 = assert_close(out, o32, f"{label} vs fp32 CPU layer")
    print(f"{label}: ids exact; vs f64 max-abs {m64[0]:.2e} rel-L2 {m64[1]:.2e}; "
          f"vs f32 max-abs {m32[0]:.2e} rel-L2 {m32[1]:.2e}", flush=True)
    return out, ids, w
