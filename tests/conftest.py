"""Test configuration.

Markers: `gpu` tests need a HIP device and the built HIP library; they run
with `pytest -m gpu` on a GPU host.  Everything else runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def hip():
    """One HIP context for the whole GPU session (device 0)."""
    from sharpinference_amd import native
    ctx = native.HipContext(0)
    yield ctx
    ctx.close()
