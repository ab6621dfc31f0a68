"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle and host-side checks (no GPU needed);
``-m gpu`` runs the parity tests of the HIP kernels against the oracle.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "helix-lite_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    from helix_kv import _native

    _native.lib()  # raises if the library was not built
    return torch.device("cuda:0")
