"""Shared test setup.

Markers: `gpu` tests need a ROCm GPU and the built libcrane_hip.so; everything
else runs on the CPU (oracle pins, C-ABI symbol/argument checks, host logic).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and libcrane_hip.so")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from crane_amd import _lib
    _lib.lib()  # fails loudly when the library is missing
    return torch.device("cuda:0")
