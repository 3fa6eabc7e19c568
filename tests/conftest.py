"""Test setup: import paths and the ``gpu`` marker.

``-m "not gpu"``: the oracle against the reference's golden vectors, the
repack, the host logic and the C ABI exports (no GPU needed).
``-m gpu``: the HIP path against the oracle through the C ABI (MI355X).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "amd.c_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def dev():
    """The opened device; a GPU test fails (does not skip) when it cannot open."""
    import amdc
    amdc.open_device()
    return amdc
