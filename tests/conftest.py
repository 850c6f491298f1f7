from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from __graft_entry__ import load_package  # noqa: E402


def pytest_configure(config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP kernels)")


@pytest.fixture(scope="session")
def nq():
    return load_package()


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a GPU")
    return torch.device("cuda:0")
