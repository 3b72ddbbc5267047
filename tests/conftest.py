"""Shared test setup.

Markers: `gpu` tests need an MI355X (run with `-m gpu`); everything else runs
on the CPU.  The package directory `llama.go_amd/` is not an importable
Python name, so its `llg` package is put on sys.path here.
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "llama.go_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X, gfx950)")


@pytest.fixture(scope="session")
def dev():
    """One llg.Device for the GPU session; fails loudly when the library or GPU is missing."""
    import llg

    d = llg.Device()
    yield d
    d.close()


@pytest.fixture
def rng():
    return np.random.default_rng(int(os.environ.get("LLG_TEST_SEED", "1234")))
