import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gemm():
    """The product context on cuda:0; the HIP library must load (no fallback)."""
    import torch

    from qwenny_amd import Gemm

    assert torch.cuda.is_available(), "GPU test without a GPU"
    torch.cuda.init()
    return Gemm.load(0)
