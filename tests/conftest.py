import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests' device.  Fails (does not skip) when no GPU is visible, so a
    -m gpu run can never pass vacuously."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    from gdsllm_amd import capi

    capi()  # the kernel library must be built and loadable
    return torch.device("cuda:0")
