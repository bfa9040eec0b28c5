import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box through the C ABI)")


@pytest.fixture(scope="session")
def cuda():
    """The HIP device through torch; GPU tests fail (not skip) when the product library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import kungfu_amd

    kungfu_amd.lib()
    return torch.device("cuda:0")
