"""Shared test setup: the `gpu` marker, import paths and data helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def close(a, b, rel):
    """The reference's tolerance: relative above 1, absolute below (kernels/tests.rs:52-55)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b) <= rel * np.maximum(np.maximum(np.abs(a), np.abs(b)), 1.0)
