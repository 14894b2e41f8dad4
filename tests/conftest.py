"""Shared pytest setup: the `gpu` marker, import paths and GPU fixtures.

CPU runs (`-m "not gpu"`) cover the oracle against golden vectors and
closed-form checks, the host-side binding logic and the C-ABI exports.  GPU
runs (`-m gpu`) are the parity tests: HIP kernels through the C ABI versus
the oracle on the same seeded inputs.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "oracle", ROOT / "mini-infer_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built kernels")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def mk(dev):
    """The kernel binding; fails (does not skip) when the library is missing."""
    import mi_kernels
    mi_kernels.load_library()
    return mi_kernels


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle
