import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built libejhip.so")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail loudly when it or the library is missing
    (there is no CPU path to fall back to)."""
    import torch

    import einjax_amd._lib as lib

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    lib.load()
    return torch.device("cuda", 0)
