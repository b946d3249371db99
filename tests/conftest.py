"""Shared fixtures. GPU tests carry ``@pytest.mark.gpu`` and compare the HIP kernels (called
through the C ABI) with the CPU oracle on identical seeded inputs."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("no HIP device in this environment")
    return torch.device("cuda")


def seeded(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)
