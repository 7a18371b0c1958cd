"""Shared fixtures.  GPU tests are marked @pytest.mark.gpu and call the HIP
library only through its C ABI (include/qgemv.h via ctypes)."""
from __future__ import annotations

import importlib
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__ as ge  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (runs on the MI355X box)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def rinf():
    return ge.load_package()


@pytest.fixture(scope="session")
def synth(rinf):
    return importlib.import_module(ge.PKG_NAME + ".synth")


@pytest.fixture(scope="session")
def oracle():
    return ge.load_oracle()


@pytest.fixture(scope="session")
def ctx(rinf):
    c = rinf.GpuContext(0)
    yield c
    c.close()


def normwise_err(y, ref):
    import numpy as np
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref)) if ref.size else 0.0
    if den == 0.0:
        return float(np.max(np.abs(y))) if y.size else 0.0
    return float(np.max(np.abs(y - ref)) / den)


# GEMV tolerance (1e-4, f32 accumulate, applied
# normwise: max|y - y_ref| / max|y_ref|; a per-element relative bound is
# unattainable where outputs cancel to near zero).
GEMV_TOL = 1e-4
