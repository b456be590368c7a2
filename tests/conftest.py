"""pytest configuration: the ``gpu`` marker and shared helpers.

``-m "not gpu"`` runs here (no GPU): the oracle against the compiled reference,
closed forms and golden fixtures, host-side formats, and the C ABI's symbol
table and host-side argument checks.  ``-m gpu`` runs on an MI355X: parity of
the HIP kernels (called through the C ABI) with the oracle.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (parity of the HIP kernels)")


@pytest.fixture(scope="session")
def orc():
    from oracle import binding
    binding.orc()
    return binding


@pytest.fixture(scope="session")
def dev():
    """The GPU, with the HIP library loaded (fails loudly if either is missing)."""
    import torch
    import ternocl_amd as T
    assert torch.cuda.is_available(), "no GPU visible"
    T.lib()
    return torch.device("cuda:0")
