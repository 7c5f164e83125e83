"""pytest setup: import paths, the `gpu` marker, shared fixtures.

Tests marked `gpu` need an MI355X (run with -m gpu on the GPU box); all
others run on the CPU and load libqkern.so without launching anything.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "metal-pjrt-plugin_amd"),
          os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X GPU (HIP kernels are launched)")


@pytest.fixture(scope="session")
def dev():
    """cuda:0; fails loudly (no skip) when a GPU test runs without a GPU."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before it runs, so a GPU fault still shows which test.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield
