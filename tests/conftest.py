"""Shared pytest setup: the ``gpu`` marker, import paths and small configs."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "deepseek-v3-lite_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def small_cfg():
    """The reference's small component config (tests/conftest.py:41-68), MoE keys only."""
    return {"dim": 64, "n_routed_experts": 4, "n_shared_experts": 1, "n_activated_experts": 2,
            "moe_inter_dim": 64}


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN
