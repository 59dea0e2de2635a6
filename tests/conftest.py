"""Test configuration: import paths, the `gpu` marker and shared helpers.

CPU tests (-m "not gpu") check the oracle, the host logic and the C ABI's contract
errors. GPU tests (-m gpu) run the HIP kernels through the C ABI and compare them with
the oracle on the same seeded inputs.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "wayfinder-attention_amd")
for p in (PKG_DIR, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")
