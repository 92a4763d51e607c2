"""Shared pytest setup: the ``gpu`` marker, the package import and the oracle."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle, available, build

    if not available("oracle"):
        build()
    return Oracle("oracle", threads=4)


@pytest.fixture(scope="session")
def ref():
    from oracle.oracle import Oracle, available

    if not available("ref"):
        pytest.skip("reference scalar kernels (oracle/_ref) not built on this machine")
    return Oracle("ref")


@pytest.fixture(scope="session")
def iw():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
