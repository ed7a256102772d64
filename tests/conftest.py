import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built native library")


def assert_close(actual, expected, rtol, atol_rel=1e-6, name=""):
    """|a - e| <= rtol*|e| + atol_rel*max|e| elementwise (the absolute floor
    covers exact zeros and cancellation in long fp32 sums)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    if e.size == 0:
        return
    scale = float(np.max(np.abs(e))) if e.size else 0.0
    tol = rtol * np.abs(e) + atol_rel * max(scale, 1e-30)
    err = np.abs(a - e)
    bad = err > tol
    if bad.any():
        i = int(np.argmax(err - tol))
        raise AssertionError(f"{name}: {int(bad.sum())}/{e.size} elements off; worst at flat {i}: "
                             f"got {a.flat[i]!r} want {e.flat[i]!r} (tol {tol.flat[i]:.3g}, max|ref| {scale:.3g})")


@pytest.fixture(scope="session")
def cuda_device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import bc_mamba_amd._native as nat
    nat.lib()  # fail loudly if the library is not built
    return torch.device("cuda:0")


@pytest.fixture(params=["items", "lanes"])
def scan_kernel(request):
    """Runs a test under each depthwise scan family: the lane groups over
    items (scan.hip) and the lanes over states (scan_sl.hip), forced with
    the library's process-wide setting (bcm_set_scan_family) and restored
    afterwards."""
    import bc_mamba_amd._native as nat
    prev = nat.set_scan_family(request.param)
    yield request.param
    nat.set_scan_family(prev)
