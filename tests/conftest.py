import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libarfq.so on cuda:0)")


def rel_err(got, want):
    """max_i |g_i - c_i| / max(|c_i|, rms(c)): the matmul gate.  A pure |c_i|
    denominator is ill-posed for near-zero outputs of random-sign sums."""
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    rms = np.sqrt(np.mean(want * want)) if want.size else 0.0
    den = np.maximum(np.abs(want), max(rms, 1e-30))
    return float(np.max(np.abs(got - want) / den)) if want.size else 0.0


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def gpu_ctx():
    import arf_amd
    ctx = arf_amd.Context(0)
    yield ctx
    ctx.close()
