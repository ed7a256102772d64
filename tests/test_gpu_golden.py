"""The HIP path, called through the drop-in API, reproduces the committed
golden fixtures (tests/golden/*.npz): indices bit-exact, outputs and every
gradient within rtol 1e-4 (fp32) plus an absolute floor of 1e-6 * max|ref|."""
import os

import numpy as np
import pytest
import torch

from bc_mamba_amd import e_model
from bc_mamba_amd import extract_events_cuda as ee
from bc_mamba_amd.selective_scan_interface import selective_scan_flat_ch_fn
from conftest import ROOT, assert_close

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(ROOT, "tests", "golden")
PATH_CASES = ["cfg0_slice", "edges", "multi_chunk", "clamped", "z_gate"]
RTOL, ATOL_REL = 1e-4, 1e-6


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", PATH_CASES)
def test_path_reproduces_golden(cuda_device, name):
    f = load(name)
    dev = cuda_device
    T = lambda k, grad=False: torch.from_numpy(f[k]).to(dev).requires_grad_(grad)
    B, D, L = f["membrane"].shape
    x_conv = T("x_conv", True)
    params = [T(n, True) for n in ("dt_idle", "dt_active", "A", "W_B", "W_C", "D_skip")]
    z = T("z", True) if "z" in f else None
    ch, t, k, cu, counts, ms = ee.extract_base_events(T("membrane"), float(f["threshold"]))
    for got, key in ((ch, "ch"), (t, "t"), (k, "k"), (cu, "cu"), (counts, "counts")):
        assert got.dtype == torch.int32 and np.array_equal(got.cpu().numpy(), f[key]), key
    assert int(ms) == int(f["max_seqlen"])
    u = e_model.GatherEventsFn.apply(x_conv, ch, t)
    assert np.array_equal(u.detach().cpu().numpy(), f["u"])  # a gather is a copy: exact
    y, x = selective_scan_flat_ch_fn(u, k, cu, int(ms), *params[:5], D=params[5], z=z, is_depthwise_bc=True)
    assert_close(y.detach().cpu(), f["y_z"] if z is not None else f["y"], RTOL, ATOL_REL, "y")
    assert_close(x.cpu(), f["x"], RTOL, ATOL_REL, "x")
    out = e_model.restore_dense_fn(y, t, cu, D, L)
    assert_close(out.detach().cpu(), f["out"], RTOL, ATOL_REL, "out")
    out.backward(T("dout"))
    assert_close(x_conv.grad.cpu(), f["dx"], RTOL, ATOL_REL, "dx_conv")
    for p, n in zip(params, ("ddt_idle", "ddt_active", "dA", "dW_B", "dW_C", "dD")):
        assert_close(p.grad.cpu(), f[n], RTOL, ATOL_REL, n)
    if z is not None:
        assert_close(z.grad.cpu(), f["dz"], RTOL, ATOL_REL, "dz")


def test_expand_reproduces_golden(cuda_device):
    f = load("expand2")
    B, Dm, L = f["membrane"].shape
    ch, t, k, cu, counts, ms = ee.extract_base_events(torch.from_numpy(f["membrane"]).to(cuda_device),
                                                      float(f["threshold"]))
    ech, et, ek, ecu, ems = ee.expand_base_events(ch, t, k, cu, B, Dm, int(f["expand"]))
    for got, key in ((ech, "e_ch"), (et, "e_t"), (ek, "e_k"), (ecu, "e_cu")):
        assert np.array_equal(got.cpu().numpy(), f[key]), key
    assert int(ems) == int(f["e_max_seqlen"])
