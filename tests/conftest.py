import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "phi-agent_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: full-size case (seconds on the GPU)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def lib():
    import phi_qlinear

    return phi_qlinear.load()


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle
