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


class _Knobs:
    """Launch knobs set through kf_hip_set_knob for one test; each touched knob gets its old value back afterwards."""

    def __init__(self):
        self.saved = {}

    def setenv(self, name, value):
        import kungfu_amd

        if name not in self.saved:
            self.saved[name] = kungfu_amd.get_knob(name)
        kungfu_amd.set_knob(name, int(value))

    def delenv(self, name, raising=False):
        import kungfu_amd

        if name not in self.saved:
            self.saved[name] = kungfu_amd.get_knob(name)
        kungfu_amd.set_knob(name, None)

    def restore(self):
        import kungfu_amd

        for name, v in self.saved.items():
            kungfu_amd.set_knob(name, v)


@pytest.fixture
def knobs():
    k = _Knobs()
    yield k
    k.restore()
