"""Test setup: import paths, the `gpu` marker, shared fixtures.

CPU tests (`-m "not gpu"`) cover the oracle against the reference's known answers and golden vectors, the host
logic, the kernel geometry replays, and that libpaia_gemv.so loads and exports every declared symbol.
GPU tests (`-m gpu`) are the parity tests proper: they call the HIP library through its C ABI (and the torch ops) and
compare with the CPU oracle on the same seeded inputs.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "paia-project_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def gemv_lib():
    """The HIP library through its C ABI. On a GPU box a missing library is an error, never a skip."""
    from paia_gemv import load_lib
    return load_lib()


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU: run with -m gpu only on the MI355X box")
    return torch.device("cuda:0")
