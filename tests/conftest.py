"""Test tiers: `-m "not gpu"` runs here (oracle vs pinned vectors, the host
runtime through the host-check build, ABI exports); `-m gpu` runs on an
MI355X and calls libkcmm.so through its C ABI."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libkcmm.so")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    if not oracle.LIB_PATH.exists():
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def hostcheck_lib():
    from lattice_amd import build as b
    if not b.HOSTCHECK_LIB.exists():
        b.build_hostcheck()
    from lattice_amd.bindings import KcmmLibrary
    return KcmmLibrary(b.HOSTCHECK_LIB)


@pytest.fixture(scope="session")
def gpu_lib():
    """The product library on a real GPU; fails loudly when it is missing."""
    import torch
    from lattice_amd.bindings import KcmmLibrary, DEFAULT_LIB
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    assert DEFAULT_LIB.exists(), f"{DEFAULT_LIB} not built (python -m lattice_amd.build)"
    return KcmmLibrary(DEFAULT_LIB)


@pytest.fixture
def tunables(gpu_lib, monkeypatch):
    """Sets KCMM_* tuning variables for one test.  The library reads them once
    per process, so every change, and the restore after the test, is
    followed by kcmm_reload_tunables."""
    class _Tunables:
        def setenv(self, name, value):
            monkeypatch.setenv(name, value)
            gpu_lib.reload_tunables()

        def delenv(self, name):
            monkeypatch.delenv(name, raising=False)
            gpu_lib.reload_tunables()

    yield _Tunables()
    monkeypatch.undo()
    gpu_lib.reload_tunables()
