import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running test")


@pytest.fixture(scope="session")
def gpu():
    """Initialise the HIP library on cuda:0 (the attention kernels run on torch's current stream)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from llmgen_amd.attention import init_device

    init_device()
    return torch.device("cuda:0")
