"""pytest configuration: the `gpu` marker and shared helpers."""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) GPU")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda", 0)


@pytest.fixture
def decode_kernel(request):
    """Run the test with the quantized decode's kernel chosen by the test's
    `decode_kernel` parameter (indirect parametrization: "auto",
    "persistent" or "one-item"); the automatic choice is restored afterwards,
    also when the test fails."""
    from carrykernel_amd import _native
    which = {"auto": _native.DECODE_KERNEL_AUTO, "persistent": _native.DECODE_KERNEL_PERSISTENT,
             "one-item": _native.DECODE_KERNEL_ONE_ITEM}[getattr(request, "param", "auto")]
    _native.set_decode_kernel(which)
    try:
        yield which
    finally:
        _native.set_decode_kernel(_native.DECODE_KERNEL_AUTO)
