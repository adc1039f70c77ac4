"""pytest setup: import paths and the `gpu` marker.

CPU tests (`-m "not gpu"`) cover the oracle against golden vectors, the host
planner / page pool through the C ABI, and the library's exported symbols.
GPU tests (`-m gpu`) run the HIP kernels through the C ABI and compare them
with the oracle.
"""

import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "paged-attention_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (gfx950)")


@pytest.fixture(scope="module")
def gpu_device():
    """GPU test modules use this (via pytestmark): a device must be present and
    the HIP library loaded; nothing falls back to the CPU."""
    import torch

    import pa_amd
    assert torch.cuda.is_available(), "GPU tests need a device"
    pa_amd._lib.load()
    yield
