"""Test configuration: import paths and the ``gpu`` marker.

CPU tests (``-m "not gpu"``) cover the oracle against golden fixtures and closed
forms, the host-side API, and the C ABI's exports and host validation.  GPU tests
(``-m gpu``) are the parity tests proper: HIP kernels through the C ABI against
the oracle on the same seeded inputs.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "pope-pytorch_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (runs the HIP kernels)")


@pytest.fixture
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch.device("cuda")
