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
    # the host-sanitizer run of the C ABI tests (test_abi_asan.py) points the binding at its build
    lib_override = os.environ.get("POPE_AMD_TEST_LIB")
    if lib_override:
        from pope_amd import _lib
        _lib.LIB_PATH = lib_override


@pytest.fixture
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch.device("cuda")
