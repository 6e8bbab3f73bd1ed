"""Shared fixtures.  GPU tests carry @pytest.mark.gpu and use the `ctx`
fixture, which skips when no HIP device is visible (so a plain local run of
the whole suite still passes); the driver selects them with -m gpu."""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


@pytest.fixture(scope="session")
def ctx():
    import gadeon_amd as ga
    if ga.device_count() == 0:
        pytest.skip("no HIP device visible")
    c = ga.Context(0)
    yield c
    c.close()


def rel_diff(a, b) -> float:
    """Norm-wise relative error max|a-b| / max|b| (MetalSelfTest.swift:437-448)."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    mag = np.max(np.abs(b)) if b.size else 0.0
    d = np.max(np.abs(a - b)) if b.size else 0.0
    return d / mag if mag > 0 else d
