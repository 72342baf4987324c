"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs the oracle pins, the split plan, the host-side checks and
the C-ABI export check on a machine without a GPU. `-m gpu` runs the HIP
kernels against the oracle on a ROCm device.
"""

import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "baby-vllm_amd"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
