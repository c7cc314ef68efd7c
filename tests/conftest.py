import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "distributed-training_amd"
GOLDEN = ROOT / "tests" / "golden"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libdtmi.so")


def _has_gpu() -> bool:
    if os.environ.get("DTMI_FORCE_NO_GPU"):
        return False
    return Path("/dev/kfd").exists()


@pytest.fixture(scope="session")
def dev():
    """The initialised libdtmi (device 0). GPU tests fail loudly if it is missing."""
    if not _has_gpu():
        pytest.skip("no GPU in this environment")
    from dtmi import _lib
    return _lib.lib()


@pytest.fixture(scope="session")
def golden():
    def load(name):
        return np.load(GOLDEN / name, allow_pickle=False)
    return load
