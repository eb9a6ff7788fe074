"""Shared test setup.

Markers: ``gpu`` tests need a HIP device.  Without one they are skipped,
unless FAIL_WITHOUT_GPU is set, which turns the absence into a failure
(the same switch the reference's test patch offers for its device marker:
packages/torchcodec-xpu/patches/0001-Add-XPU-support-to-tests.patch:50-55).
"""

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO / "torchlib-xpu_amd", REPO / "oracle", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


def _gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    if os.environ.get("FAIL_WITHOUT_GPU"):
        return
    skip = pytest.mark.skip(reason="no HIP device (set FAIL_WITHOUT_GPU=1 to fail instead)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a HIP device")
    import mx_fbgemm  # noqa: F401  (registers torch.ops.fbgemm.*)

    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _no_lookback_faults(request):
    """After every GPU test: no sort or scan look-back wait gave up (the
    kernels report one through a host-visible word of the device)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import torch

    if not torch.cuda.is_available():
        return
    import mx_fbgemm  # noqa: F401

    assert torch.ops.mx_fbgemm.pending_lookback_faults(0) == 0, \
        "a look-back wait of the sort or a scan gave up during this test"
