"""Shared pytest setup: the `gpu` marker, import paths and fixtures."""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "pocket-workbench-android_amd"
for p in (REPO, PKG):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def pih():
    import pocketinfer_hip
    pocketinfer_hip.load_library()
    return pocketinfer_hip


@pytest.fixture(scope="session")
def backend(pih):
    b = pih.HipBackend(0)
    yield b
    b.close()


def lcg(state):
    """The reference tests' LCG (tests/quant_layout.rs:137-140)."""
    state = (state * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
    return state, state >> 33
