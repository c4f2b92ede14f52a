"""CPU checks of the C-ABI boundary: the HIP library loads without a GPU and
exports every symbol include/ingot_moe.h declares; host-only entry points
(geometry, matrix validation) follow the reference; no compute call is made."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from ingot_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ingot_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = C.CDLL(N.MOE_LIB)
    names = declared("ingot_moe.h")
    assert len(names) > 30
    for name in names:
        assert hasattr(lib, name), name
        assert name in N.MOE_SYMBOLS, f"{name} has no ctypes binding"
    synth = C.CDLL(N.SYNTH_LIB)
    for name in declared("ingot_synth.h"):
        assert hasattr(synth, name), name
        assert name in N.SYNTH_SYMBOLS, name


# src/gguf.rs:470-491
GEOMETRY = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 8: (32, 34), 10: (256, 84), 12: (256, 144),
            13: (256, 176), 14: (256, 210), 16: (256, 66), 17: (256, 74), 18: (256, 98), 20: (32, 18),
            21: (256, 110), 22: (256, 82), 23: (256, 136), 29: (256, 56), 42: (64, 18)}


def test_geometry_table_matches_reference():
    from ingot_amd.moe import InvalidData, geometry
    for kind in range(64):
        if kind in GEOMETRY:
            assert geometry(kind) == GEOMETRY[kind]
        else:
            with pytest.raises(InvalidData):
                geometry(kind)


def test_validate_matrix_contract():
    """src/metal.rs:1602-1621: zero sizes, cols % block, stride, byte length, u32 limits."""
    from ingot_amd.moe import Q4_K, InvalidData, Matrix
    ok = Matrix(np.zeros(2 * 3 * 1152, np.uint8), 2048, 3, 2, Q4_K, 1152)
    ok.validate()
    bad = [Matrix(ok.data, 2048, 3, 2, Q4_K, 1151), Matrix(ok.data, 2000, 3, 2, Q4_K, 1152),
           Matrix(ok.data, 2048, 0, 2, Q4_K, 1152), Matrix(ok.data[:-1], 2048, 3, 2, Q4_K, 1152),
           Matrix(ok.data, 2048, 3, 2, 7, 1152), Matrix(ok.data, 2048, 3, 3, Q4_K, 1152)]
    for m in bad:
        with pytest.raises(InvalidData):
            m.validate()


def test_status_strings_and_supported_kinds():
    lib = N.moe_lib()
    for st in range(5):
        assert lib.ingot_status_string(st)
    # every type of the reference's geometry table (src/gguf.rs:470-491) has kernels
    assert [k for k in range(64) if lib.ingot_kind_supported(k)] == \
        [0, 1, 2, 8, 10, 12, 13, 14, 16, 17, 18, 20, 21, 22, 23, 29, 30, 42]


def test_oracle_and_product_agree_on_validation(oracle):
    from ingot_amd.moe import Q8_0, Matrix
    for stride in (33, 34, 35):
        m = Matrix(np.zeros(4 * 34, np.uint8), 32, 4, 1, Q8_0, stride)
        ok = N.moe_lib().ingot_validate_matrix(C.byref(m.c())) == 0
        assert ok == oracle.validate(m) == (stride == 34)
