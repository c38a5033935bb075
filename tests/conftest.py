import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "bsscl-gbm_amd"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU")


@pytest.fixture(scope="session")
def engine():
    """One engine for the GPU session (every GPU test shares the device)."""
    from bsscl_gbm import _native
    if _native.device_count() < 1:
        pytest.fail("no HIP device visible for a gpu-marked test")
    eng = _native.Engine(0)
    yield eng
    eng.close()


def make_data(n, F, seed=0, nan_frac=0.0, dtype=np.float32, nan_cols=None):
    """Synthetic binary data: X ~ N(0,1), y ~ Bernoulli(sigmoid(X@w))."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, F)).astype(dtype)
    w = rng.standard_normal(F)
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-(X.astype(np.float64) @ w)))).astype(np.int64)
    if nan_frac > 0:
        cols = range(F) if nan_cols is None else nan_cols
        for j in cols:
            X[rng.random(n) < nan_frac, j] = np.nan
    return X, y
