"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs the oracle pins, the split plan, the host-side checks and
the C-ABI export check on a machine without a GPU. `-m gpu` runs the HIP
kernels against the oracle on a ROCm device.
"""

import os
import sys
import zlib

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "baby-vllm_amd"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(autouse=True)
def _seed_per_test(request):
    """Every test starts from a seed of its own (from its node id), so inputs drawn
    without an explicit generator are the same on every run."""
    import torch

    seed = zlib.crc32(request.node.nodeid.encode())
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)
