"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` tests run anywhere (oracle, host logic, ABI exports).
``-m gpu`` tests need a HIP device; they fail (not skip) without one, so a
GPU run can never pass on a missing device.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "shadow-infer_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP (MI355X) device")


@pytest.fixture(scope="session")
def dev():
    import torch

    assert torch.cuda.is_available(), "GPU test run without a HIP device"
    return torch.device("cuda:0")
