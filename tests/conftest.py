from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running CPU oracle case")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import Reference
    if not Reference.available():
        pytest.skip("oracle/_ref not built (the reference is not mounted here)")
    return Reference()


@pytest.fixture(scope="session")
def ref_opt():
    """The compiled reference where oracle/_ref is built, else None (for tests
    whose other checks stand without it)."""
    from oracle import Reference
    return Reference() if Reference.available() else None


@pytest.fixture(scope="session")
def synth():
    from util import load_synth
    return load_synth()


@pytest.fixture(scope="session")
def sa():
    """The HIP library; on a GPU run a missing library or device is an error, not a skip."""
    import torch
    from util import load_pkg
    if not torch.cuda.is_available():
        raise RuntimeError("GPU test without a visible GPU")
    mod = load_pkg()
    mod.lib()
    return mod
