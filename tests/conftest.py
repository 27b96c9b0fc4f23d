"""Shared pytest configuration.

Marker ``gpu``: needs a ROCm device (run with ``-m gpu`` on the MI355X box).
Everything else runs on the CPU.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: requires a ROCm GPU (MI355X)")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.build()
    return oracle


def _gpu_ready() -> bool:
    try:
        import torch

        return bool(torch.version.hip) and torch.cuda.device_count() > 0
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def gpu():
    if not _gpu_ready():
        pytest.fail("GPU test selected but no ROCm device is visible")
    import torch

    from fused_cpp_amd import cabi

    cabi.lib()
    torch.cuda.init()
    return torch.device("cuda", 0)
