import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on the HIP path)")


@pytest.fixture(scope="session")
def gpu():
    """Session fixture for GPU tests: fails loudly when the HIP library or the device is missing."""
    import torch

    import dirktensor_amd as dt
    from dirktensor_amd import _capi

    assert dt.LIB_PATH.exists(), f"{dt.LIB_PATH} not built: run python -m dirktensor_amd.build_ext"
    _capi.lib()
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch.device("cuda:0")
