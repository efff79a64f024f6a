"""Test configuration: the ``gpu`` marker and import paths.

``saint-llm_amd`` holds the ``saint_kv`` package; the repo root holds the CPU
oracle.  GPU tests compare the HIP library with the oracle on seeded inputs.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "saint-llm_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libsaintkv.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but no ROCm GPU is visible")
    from saint_kv import _lib

    _lib.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")
