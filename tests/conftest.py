import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rust-fp4-blackwell_amd")
ORACLE = os.path.join(ROOT, "oracle")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: long-running parity case")


@pytest.fixture(scope="session")
def orc():
    import pyoracle

    pyoracle.lib()
    pyoracle.set_threads(0)
    return pyoracle


@pytest.fixture(scope="session")
def rf():
    """The HIP library, initialised on device 0 (GPU tests only)."""
    import rfp4

    rfp4.init(0)
    return rfp4


@pytest.fixture(scope="session")
def stream(rf):
    return rf.Stream()


def reference_rel_err(y, ref):
    """The reference's metric: |d| / max(|ref|, 1e-3) (fp4_gemv/src/main.rs:165-166)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)
