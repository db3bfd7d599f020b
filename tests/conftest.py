"""Test configuration: import paths, the `gpu` marker, shared helpers.

GPU tests (marked `gpu`) call the HIP path through soinfer._C / the C ABI and
compare with the CPU oracle (oracle/oracle.py). CPU tests cover the oracle
itself against golden vectors and closed forms, the host-side Python, and
the C ABI library's exports.
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "sparse-offload-infer_amd"
for p in (str(PKG), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_sessionstart(session):
    """A fresh checkout has no built libraries (they are not committed): build them in-tree once, before any test
    imports soinfer. An existing build is used as it is."""
    from __graft_entry__ import ensure_built

    ensure_built()


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    torch.use_deterministic_algorithms(True)
    return torch.device("cuda:0")
