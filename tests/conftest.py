import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def hip_hooks():
    """Set the HIP library's test hooks for one test: hip_hooks("FORCE_LUT", ...);
    the previous bits come back at teardown."""
    from qflash_amd import _lib

    prev = []

    def set_(*names):
        old = _lib.set_test_hooks(*names)
        if not prev:
            prev.append(old)
    yield set_
    if prev:
        _lib.load().qflash_hip_set_test_hooks(prev[0])
