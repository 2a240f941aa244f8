"""pytest configuration: import paths, the ``gpu`` marker and shared fixtures.

CPU tests (``-m "not gpu"``) check the oracle against the reference's known
answers and closed forms, the C-ABI library's exports and the fronts' contract
checks. GPU tests (``-m gpu``) run the HIP kernels through the fronts / C ABI
and compare them with the oracle on the same seeded inputs.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "koemi-5hom_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built kernel library")


@pytest.fixture(scope="session")
def device():
    """cuda:0 with the kernel library loaded; GPU tests fail (not skip) without it."""

    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device (torch.cuda.is_available() is False)"
    from koemi_amd import _native

    _native.load_library()
    return torch.device("cuda:0")
