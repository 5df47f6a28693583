"""Shared test setup: the `gpu` marker and import paths.

CPU tests (-m "not gpu") cover the oracle against the golden vectors, the host
logic and the C ABI's symbol table.  GPU tests (-m gpu) call libmoehip.so
through its C ABI and compare with the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "moe.cc_amd"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libmoehip.so")


def gpu_present() -> bool:
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def moehip():
    """The product library, initialised on device 0 (GPU tests only)."""
    import moehip as M
    M.init(0)
    return M
