import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the gfx950 kernels)")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment (run with -m gpu on the GPU box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True, scope="session")
def _check_bounded_waits():
    """Every requantizing GEMM and Gram product of a GPU test checks its
    bounded-wait status word: a wait that ran out fails the test
    (PratchyaWaitTimeout) instead of leaving NaN outputs."""
    if not _gpu_available():
        yield
        return
    from pratchya_amd import _kernels
    prev = _kernels.check_waits(True)
    yield
    _kernels.check_waits(prev)
