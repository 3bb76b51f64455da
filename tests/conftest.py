import os
import sys

# the tests force launch plans through the VYBDQ_* tuning variables, which the library reads only
# when VYBDQ_TUNING is set before its first launch
os.environ.setdefault("VYBDQ_TUNING", "1")

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
