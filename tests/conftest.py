"""Test configuration: the `gpu` marker and repository import paths.

Tests marked ``gpu`` need an MI355X (they call the HIP library through its
C ABI); everything else runs on the CPU and exercises the oracle, the host
logic and the library's exported symbols without launching GPU work.
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.ensure_built()
    return oracle


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def jasper():
    if not gpu_available():
        pytest.skip("no GPU")
    import jasper_amd
    jasper_amd._load_lib()
    return jasper_amd
