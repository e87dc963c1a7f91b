import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "gl-sdm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity tests of the native path")


def has_gpu():
    import torch
    return torch.cuda.is_available()


@pytest.fixture
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _commit_status_checks(request):
    """GPU tests run with the commit status check on: every commit-family call
    reads its device status words and raises if the sort failed."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    from glsdm import _native
    prev = _native.set_checks(status=True)
    try:
        yield
    finally:
        _native.set_checks(**prev)
