import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def kernel_options():
    """Set kernel-variant options of the library (fmoe_set_option) for one test; the previous
    values come back at teardown.  Usage: ``kernel_options(plan=1, bwd_fused=1)``."""
    from fastmoe_amd import _abi

    saved = {}

    def set_options(**values):
        for k, v in values.items():
            prev = _abi.set_option(k, v)
            saved.setdefault(k, prev)

    yield set_options
    for k, v in saved.items():
        _abi.set_option(k, v)
