import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu_lib():
    """The loaded HIP library; GPU tests fail (not skip) if it cannot load."""
    import torch
    assert torch.cuda.is_available(), "GPU test selected but no GPU visible"
    from qllm2_amd import _lib
    return _lib.lib()
