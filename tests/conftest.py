import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "laguna-raw-halo-strix_amd")
for p in (PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X / gfx950)")


@pytest.fixture(scope="session")
def golden():
    with np.load(os.path.join(ROOT, "tests", "golden", "golden.npz")) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def ctx():
    """Device context for GPU tests.  Skips only when the host has no HIP device;
    a missing or unloadable library is an error, never a skip."""
    import laguna_hip as lh

    lh.lib()  # raises if liblaguna_hip.so is missing
    if lh.device_count() == 0:
        pytest.skip("no HIP device on this host")
    return lh.VulkanContext(0)


def parity(y, y64, absdot, tol=1e-4):
    """The two parity metrics: max_i |y-yhat| / sum_j |W_ij x_j| and
    ||y-yhat||_inf / ||yhat||_inf, with yhat the f64 accumulation."""
    y = np.asarray(y, np.float64)
    err = np.abs(y - y64)
    m1 = float(np.max(err / np.maximum(absdot, 1e-300))) if y.size else 0.0
    m2 = float(np.max(err) / max(np.max(np.abs(y64)), 1e-300)) if y.size else 0.0
    assert np.all(np.isfinite(y)), "non-finite outputs"
    assert m1 <= tol and m2 <= tol, f"parity: max|err|/sum|wx| = {m1:.3e}, |err|inf/|y|inf = {m2:.3e} (tol {tol})"
    return m1, m2
