"""Test configuration.

Markers: ``gpu`` tests need an MI355X (they run through libingot_moe.so, the
C ABI); everything else runs on the CPU (the oracle against the reference's
known answers and golden fixtures, host logic, and that the C-ABI library
loads and exports every declared symbol).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (gfx950) and the built libingot_moe.so")


@pytest.fixture(scope="session")
def gpu():
    from ingot_amd.moe import Gpu
    import gc
    g = Gpu(0)
    yield g
    gc.collect()  # layers the tests dropped are destroyed before their context
    g.close()


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle
    pyoracle.lib()
    return pyoracle
