import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def pkg():
    """The product package (glm5-on-v100_amd/, imported as glm5_on_v100_amd)."""
    import __graft_entry__

    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def lib(pkg):
    """The loaded C-ABI library; raises if it was not built."""
    return pkg.load_library()


@pytest.fixture(scope="session")
def ops(pkg, lib):
    return pkg._sm70_ops


@pytest.fixture(scope="session")
def dev():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")
