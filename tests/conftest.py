"""Shared fixtures. `gpu`-marked tests need an MI355X; everything else runs on CPU."""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X / gfx950) and the built libq4mi.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle import q4_oracle
    return q4_oracle


@pytest.fixture(scope="session")
def pkg():
    """The product package (its directory name is not an identifier)."""
    return importlib.import_module("openflowlm-next_amd")


@pytest.fixture(scope="session")
def lib(pkg):
    return pkg.load_library()


@pytest.fixture(scope="session")
def gpu(pkg):
    """A GPU device; the native library must load (no fallback exists)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    pkg.load_library()          # raises if libq4mi.so was not built
    return torch.device("cuda", 0)


def say(msg: str) -> None:
    """Name the case before a GPU step, flushed, so a fault is attributable."""
    print(f"[case] {msg}", flush=True)


@pytest.fixture
def rng():
    return np.random.default_rng(0)
