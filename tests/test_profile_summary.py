"""Host logic of the rocprofv3 summaries bench.py reads (ingot_amd.profile_summary)."""
import os
import sys

from ingot_amd.profile_summary import _short_mangled, stage_kernel

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_stage_kernel_names():
    assert stage_kernel("void ingot::k_gemm_f16<12, true, 0, 128>(unsigned char const*)") == "k_gemm_f16<gate_up>"
    assert stage_kernel("void ingot::k_gemm_f16<18, false, 0, 64>(unsigned char const*)") == "k_gemm_f16<down>"
    assert stage_kernel("void ingot::k_gemm<8, true>(unsigned char const*)") == "k_gemm<gate_up>"
    assert stage_kernel("void ingot::k_router_t<8, 16>(float const*)") == "k_router"
    assert stage_kernel("ingot::k_dec_gate_up2<12, 1, 3, 1, 2>(unsigned char const*)") == "k_dec_gate_up2"
    assert stage_kernel("ingot::k_combine(float const*)") == "k_combine"
    m = "_ZN5ingot10k_gemm_f16ILi12ELb1ELi0ELi128EEEvPKhS2_S2_S2_jmmjjPKDF16_S4_PKfPKjjS8_jfPfPDF16_SA_S9_jjS6_PjSB_"
    assert _short_mangled(m) == "ingot::k_gemm_f16<12, true, 0, 128>"
    assert stage_kernel(m) == "k_gemm_f16<gate_up>"
    assert _short_mangled("_ZN5ingot10k_dispatchEPKjjjjjPjS2_S2_S2_S2_jjPKfmPDF16_S5_PfjS4_jS2_j") == "ingot::k_dispatch"


def test_bench_reads_committed_traffic():
    """Every committed PMC summary carries per-kernel traffic lines that bench.py finds."""
    sys.path.insert(0, ROOT)
    import bench
    assert bench.measured_traffic("k_gemm_f16<gate_up>", "c1 prefill512")[0] > 0
    assert bench.measured_traffic("k_dec_gate_up2", "c0 b=1")[0] > 0
    assert bench.measured_traffic("no_such_kernel", "c0 b=1") == (None, None)
