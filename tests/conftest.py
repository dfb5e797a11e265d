import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsumma_amd.so)")


@pytest.fixture(autouse=True)
def _fixed_global_rng():
    """Each test starts from the same torch and numpy global generator state, so
    its unseeded random inputs do not depend on which tests ran before it."""
    import numpy as np
    import torch

    torch.manual_seed(1234)
    np.random.seed(1234)


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import summa_amd

    summa_amd.lib()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")
