"""Shared test configuration.

Markers: `gpu` = needs an MI355X (runs on the GPU box via `pytest -m gpu`);
everything else runs on the CPU. The oracle (oracle/) is the checker for
both; the HIP library (pulsar_amd/libpulsar_moe.so) is what GPU tests call.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

REFERENCE = Path(os.environ.get("PULSAR_REFERENCE", "/root/reference"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu)")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def dev():
    """torch + the HIP library on cuda:0 (skips when no GPU is visible)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from pulsar_amd import _lib

    _lib.load()
    return torch.device("cuda:0")
