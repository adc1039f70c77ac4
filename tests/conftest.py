"""pytest setup: import paths and the `gpu` marker.

CPU tests (`-m "not gpu"`) cover the oracle against golden vectors, the host
planner / page pool through the C ABI, and the library's exported symbols.
GPU tests (`-m gpu`) run the HIP kernels through the C ABI and compare them
with the oracle.
"""

import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "paged-attention_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (gfx950)")
