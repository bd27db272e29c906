"""Shared pytest setup.

Markers: `gpu` tests need an MI355X (gfx950) and run through libnerf.so's C ABI;
everything else runs on the CPU (oracle pinning, host logic, library load).
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950); parity tests through the C ABI")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def lib():
    from nerf_amd import _lib

    return _lib.load()


def announce(msg: str) -> None:
    """Names the GPU case about to run, flushed, so a crash log identifies it."""
    print(f"[case] {msg}", flush=True)
