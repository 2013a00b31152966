import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "distributed-hipkittens_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def hk():
    """The native path; on a GPU box a missing build is an error, not a skip."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import hkmoe
    return hkmoe
