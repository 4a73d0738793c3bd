"""Test configuration.

`gpu` tests need a gfx950 device and libmoe_hip.so; everything else runs on
the CPU (oracle pinning, host logic, the C ABI's exported surface).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "llama-rs-metal_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    # No fallback: a GPU test fails loudly if the HIP library or the device
    # is missing.
    from hip_backend import Gpu

    g = Gpu()
    print(f"[gpu] {g.name}", flush=True)
    yield g
    g.close()
