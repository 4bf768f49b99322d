"""Shared test configuration: the ``gpu`` marker and numeric helpers."""

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X and the built libkx355.so")


@pytest.fixture(scope="session")
def device():
    """The GPU for ``gpu`` tests. The library must be built: a missing library fails, it does
    not skip."""
    import torch

    from kinomlx_amd import _lib

    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible GPU")
    _lib.load()
    return torch.device("cuda:0")


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64))))


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-300))


os.environ.setdefault("PYTHONHASHSEED", "0")
