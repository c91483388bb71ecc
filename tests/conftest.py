import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C ABI")


@pytest.fixture(scope="session")
def torch_gpu():
    """torch with a visible GPU. torch is imported before libapk.so is loaded
    so that both share one HIP runtime (same libamdhip64 SONAME)."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but no GPU is visible")
    return torch


@pytest.fixture(scope="session")
def apk(torch_gpu):
    import apk_amd
    apk_amd.load()
    return apk_amd
