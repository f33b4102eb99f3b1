from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO_ROOT = Path(__file__).resolve().parent.parent
if str(REPO_ROOT) not in sys.path:
    sys.path.insert(0, str(REPO_ROOT))

import __graft_entry__  # noqa: E402


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (HIP) device; CPU runs deselect with -m 'not gpu'"
    )


def pytest_runtest_setup(item: pytest.Item) -> None:
    """A GPU test fails without a GPU, so a run can only pass by running it."""
    if item.get_closest_marker("gpu"):
        import torch

        if not torch.cuda.is_available():
            pytest.fail("needs a GPU; on a CPU-only machine run pytest -m 'not gpu'", pytrace=False)


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")
