"""pytest configuration: the `gpu` marker and import paths.

CPU tests (``-m "not gpu"``) cover the oracle against the reference's known
answers and the committed golden vectors, the host-side mirror, and the C ABI
surface of libforge_hip.so without touching a GPU.  GPU tests (``-m gpu``) are
the parity tests proper: they call the HIP library through the C ABI and
compare with the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "forge-lm_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    return O


@pytest.fixture(scope="session")
def fhp():
    import forge_hip
    return forge_hip
