import os
import sys

import zlib

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long CPU test")


@pytest.fixture(scope="session")
def hip():
    """The kernel library; GPU tests fail (not skip) when it or the device is missing."""
    from quicklm_amd import hip as H

    H.lib()
    n = H.device_count()
    assert n > 0, "no HIP device visible"
    print(f"[gpu] {H.device_name()}", flush=True)
    return H


@pytest.fixture(scope="session")
def orc():
    from oracle.oracle import Oracle

    o = Oracle()
    o.set_threads(min(16, os.cpu_count() or 1))
    return o


@pytest.fixture
def rng(request):
    """Seeded from the test's name with CRC-32 (str hash() is salted per
    process), so every run of a test draws the same inputs."""
    seed = zlib.crc32(request.node.name.encode())
    return np.random.default_rng(seed)
