import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C ABI)")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 after checking the HIP library loads and the device is gfx950."""
    import torch

    import deepfuse_amd as df

    assert torch.cuda.is_available(), "GPU test without a GPU"
    torch.cuda.set_device(0)
    df.lib()
    assert df.lib().df_device_arch_ok() == 1, "device is not gfx950"
    return torch.device("cuda:0")
