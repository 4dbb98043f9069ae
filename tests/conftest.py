import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device for parity tests. Fails (does not skip) without one: the GPU tier must
    run the HIP kernels, never something else."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from ancha_amd import fused

    assert fused.available(), "the gfx950 kernel library does not run on this device"
    return torch.device("cuda:0")
