import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP path")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Session fixture for GPU tests: a GPU test must never pass silently on CPU."""
    if not gpu_available():
        pytest.skip("no GPU in this process (GPU tests run on the MI355X box)")
    import grout_amd

    grout_amd.lib()  # raises if the HIP library is missing
    return grout_amd
