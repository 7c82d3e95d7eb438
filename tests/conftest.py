"""Shared test setup.

Markers: `gpu` tests need an MI355X and call the HIP library through its C
ABI; everything else runs on the CPU.
"""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "recursive-routing-racer-rs_amd")
for p in (REPO, PKG, os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs through the HIP C ABI)")


def _ensure_host_libs():
    # The oracle and the input generator are plain C: build them if absent.
    if not os.path.exists(os.path.join(REPO, "oracle", "liboracle.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle")], check=True)
    if not os.path.exists(os.path.join(PKG, "lib", "librrr_synth.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(PKG, "csrc"), "../lib/librrr_synth.so"], check=True)


_ensure_host_libs()


@pytest.fixture(scope="session")
def ctx():
    """One HIP context on device 0 for the whole GPU session."""
    import rrr_hip
    c = rrr_hip.Context(0)
    yield c
    c.close()
