"""Test configuration: import paths, the ``gpu`` marker and fixture loading."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "qpu-xla-triton_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
for path in (str(ROOT), str(PKG)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP device (runs on the MI355X box)")


def load_golden(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as data:
        return {key: data[key] for key in data.files}


@pytest.fixture
def golden():
    return load_golden
