"""Shared test configuration.

Markers: ``gpu`` marks tests that need an MI355X (run with ``-m gpu``); the
default CPU suite is ``-m "not gpu"``.  The repository root is put on
sys.path so ``oracle`` (the CPU checker) and the packages import from a
checkout.
"""
from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X GPU (HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running case")


def gpu_available() -> bool:
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.build()
    return oracle
