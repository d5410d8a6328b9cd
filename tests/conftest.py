"""pytest configuration: the `gpu` marker and shared fixtures.

Tests marked `gpu` run the HIP kernels through libtfq's C ABI on a real
MI355X; everything else runs on the CPU (oracle pins, host logic, ABI
surface). The oracle under oracle/ is the checker only.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def ctx():
    from edgeexpert_amd import ops
    c = ops.Context()
    yield c
    c.close()


@pytest.fixture(scope="session")
def stream():
    from edgeexpert_amd.runtime import Stream
    return Stream()
