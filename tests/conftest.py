"""Shared pytest setup: import paths, the `gpu` marker, and the seed fixture.

Mirrors the reference's tests/conftest.py:16-21 (seed 42 before every test).
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "msda-triton_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and libmsda_hip.so")
    config.addinivalue_line("markers", "slow: full-size parity cases")


@pytest.fixture(autouse=True)
def seed_rng() -> None:
    torch.manual_seed(42)
    if torch.cuda.is_available():
        torch.cuda.manual_seed(42)


@pytest.fixture
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda")
