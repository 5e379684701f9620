"""Test configuration: the `gpu` marker, import paths, shared fixtures.

CPU tier (`-m "not gpu"`): the oracle against golden vectors and exact
checkers, host logic, and that the C ABI library loads and exports every
symbol include/fp64emu.h declares.  GPU tier (`-m gpu`): parity of the HIP
path with the oracle, through the C ABI and the torch ops.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("fp64-emu_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950)")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")
