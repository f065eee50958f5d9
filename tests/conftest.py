"""Test configuration: import paths, the ``gpu`` marker, shared fixtures.

CPU tier (``-m "not gpu"``): the oracle against the reference's known answers,
the product quantizers against the oracle's, the C ABI's exports and argument
validation, the native LRU bookkeeping.  GPU tier (``-m gpu``): parity of the
gfx950 HIP path against the oracle through the C ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "freetoken-intel_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) through ROCm")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")
