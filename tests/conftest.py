import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the HIP kernel library")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def device():
    import torch

    if not _gpu_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def backend(device):
    import torch

    from thintensor_amd.backend import HipDecodeBackend

    return HipDecodeBackend(device, torch.float16, 2048, 2048, 512, 8192)
