import os
import sys

import pytest

try:  # imported at collection so a slow first import is not charged to a test's timeout
    import torch  # noqa: F401
except ImportError:  # pragma: no cover
    torch = None

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PACKAGE_DIR = os.path.join(ROOT, "nemotron-3-embed-webgpu_amd")
for p in (ROOT, PACKAGE_DIR, os.path.join(ROOT, "oracle"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity tests through the C ABI")


def _flush_print(msg: str) -> None:
    print(msg, flush=True)


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU step so a failing run is attributable.
    if request.node.get_closest_marker("gpu"):
        _flush_print(f"\n[gpu-case] {request.node.nodeid}")
    yield


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch
