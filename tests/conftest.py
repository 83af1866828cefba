import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


@pytest.fixture
def gpu():
    """The GPU device for HIP-kernel tests. A test marked ``gpu`` fails (it
    does not skip) when no GPU or no kernel library is present, so a missing
    device or build can never pass as a green run."""
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible ROCm device")
    from astrai_amd.extension import KERNEL_NAMES, is_available
    from astrai_amd.extension.loader import load_error

    missing = [k for k in KERNEL_NAMES if not is_available(k)]
    if missing:
        pytest.fail(f"HIP kernels not loaded ({missing}): {load_error()}")
    return torch.device("cuda", 0)
