import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X / gfx950) and the built HIP library")


def _oracle_built() -> bool:
    return (ROOT / "oracle" / "liboracle_c.so").exists()


@pytest.fixture(scope="session", autouse=True)
def _build_oracle():
    """The oracle's C part is a test dependency; build it if it is missing."""
    if not _oracle_built():
        import subprocess

        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
    yield


@pytest.fixture(scope="session")
def oracle():
    from oracle import sparsepr_oracle

    return sparsepr_oracle


@pytest.fixture(scope="session")
def dev():
    """A GPU device with the HIP library loaded.  Skips only when there is no
    GPU at all; a missing library on a GPU box is a failure, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from sparsepr_amd import _lib

    _lib.load()
    return torch.device("cuda:0")

