import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def max_rel(got, want):
    """The reference's comparison: max|got - want| / max|want| (EngineTests.cs:210-211)."""
    import numpy as np
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    scale = max(float(np.abs(want).max()), 1e-30)
    return float(np.abs(got - want).max()) / scale


@pytest.fixture
def hip():
    """The default HIP backend; GPU tests fail loudly (not skip) when the native library is missing.
    Looked up per test: a test that marks the device lost leaves the next one a new backend, as
    HipBackend.Default does after a loss."""
    from simdonnx_amd.backend import HipBackend
    return HipBackend.default()
