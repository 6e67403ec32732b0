import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "torch-point-ops_amd")
for p in (REPO, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def dev():
    """The GPU device; GPU tests fail (not skip) without one."""
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("this test needs a GPU (run it on the MI355X box)")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def tpo():
    import torch_point_ops

    return torch_point_ops


@pytest.fixture(scope="session")
def O():
    from oracle import oracle

    oracle.build()
    return oracle
