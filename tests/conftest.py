import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Initialises torch (device memory / streams) and the HIP library on cuda:0."""
    import torch  # torch first: its HIP runtime is the one both sides then share

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import aether_amd as A

    A.check(A.lib().aeth_init(0), "aeth_init")
    return torch
