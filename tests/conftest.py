import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def O():
    import oracle
    return oracle.load()


@pytest.fixture(scope="session")
def R():
    """The reference's own CPU code (oracle/_ref); skipped where it was not built."""
    import oracle
    r = oracle.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference tree unavailable)")
    return r


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
