"""GPU parity of the fused restore -> out_proj op (bcm_restore_proj_fwd /
bcm_restore_proj_bwd; reference e_model.py:499-504: restore_dense_fn, then
the nn.Linear out_proj) against the float64 composition
F.linear(orc.restore_fwd(y, t, cu, D, L), W, bias) and its autograd
gradients, at the fp32 bar (rtol 1e-4, absolute floor 1e-6 * max|ref|):

  out    the projection of the zero-order hold (never formed on the GPU)
  dy     dout W summed over the steps each event owns (the restore backward)
  dW     sum over (b, t) of dout (x) z
  dbias  dout's column sums (torch)

Cases cover ragged last tiles (L % 64 != 0), d_model and D that are not
multiples of the 64 x 64 output tiles, channels without events, full
density, the expand layout of the bitmask (mask_row_div 2), and a
config-4 layer slice (d_inner 512, d_model 256, L 1024, ~7 % density).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from bc_mamba_amd import restore_dense_cuda_nodecay as rd
from conftest import assert_close
from oracle import event_path as orc

pytestmark = pytest.mark.gpu

RTOL, FLOOR = 1e-4, 1e-6


def _events(B, D, L, p, seed, mrd=1, empty_every=0):
    """Events of B*D channels from a random membrane; with mrd > 1, groups of
    mrd consecutive channels share one bitmask row (the expand layout)."""
    g = torch.Generator().manual_seed(seed)
    base = (torch.rand(B, D // mrd, L, generator=g) < p).float()
    if empty_every:
        base.view(-1, L)[::empty_every] = 0.0
    mem = base.repeat_interleave(mrd, dim=1)
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem.numpy(), 0.5)
    return base, ch, t, cu


def _index(base, t, cu, L, mrd, dev):
    """The event index (bitmask rows of the base channels, tile table of
    every channel) as the fused extraction hands it over."""
    def steps(v):  # the index builder takes a non-null step array even without events
        return torch.from_numpy(v if len(v) else np.zeros(1, np.int32)).to(dev)

    if mrd == 1:
        bm, ts = rd.build_event_index(steps(t), torch.from_numpy(cu).to(dev), L)
        return bm, ts, 1
    # bitmask of the base channels, tile table of the expanded ones
    B, Db, _ = base.shape
    bch, bt, _, bcu, _, _ = orc.extract_base_events(base.numpy(), 0.5)
    bm, _ = rd.build_event_index(steps(bt), torch.from_numpy(bcu).to(dev), L)
    _, ts = rd.build_event_index(steps(t), torch.from_numpy(cu).to(dev), L)
    return bm, ts, mrd


CASES = [  # B, D, L, d_model, density, mask_row_div
    (3, 64, 300, 32, 0.3, 1),      # ragged last tile, one partial column tile
    (2, 100, 1000, 80, 0.15, 1),   # D and d_model off the 64 grid
    (2, 64, 1100, 64, 0.2, 2),     # expand layout, two dW segments per sequence
    (1, 32, 64, 16, 1.0, 1),       # every step an event
    (2, 64, 128, 64, 0.0, 1),      # no events: out = bias, dy empty
    (4, 512, 1024, 256, 0.07, 1),  # config-4 layer slice
    (3, 64, 300, 64, 0.3, 1),      # LDS-DMA forward with an odd tile count (5 tiles: a half item pair)
    (1, 4096, 128, 64, 0.1, 1),    # dim past the DMA forward's LDS: the register-staged form runs
    (2, 100, 1024, 128, 0.2, 1),   # LDS-DMA weight gradient: two 512-step segments, a partial channel block
    (1, 192, 1056, 256, 0.1, 1),   # ... and a last segment of 32 steps, two 128-row blocks of W
]


@pytest.mark.parametrize("B,D,L,dm,p,mrd", CASES)
def test_restore_proj_matches_oracle(cuda_device, B, D, L, dm, p, mrd):
    dev = cuda_device
    print(f"restore_proj case B={B} D={D} L={L} d_model={dm} p={p} mrd={mrd}", flush=True)
    base, ch, t, cu = _events(B, D, L, p, seed=L + D + dm, mrd=mrd, empty_every=7)
    E = len(t)
    g = torch.Generator().manual_seed(3)
    y = torch.randn(E, generator=g)
    W = torch.randn(dm, D, generator=g) / np.sqrt(D)
    bias = torch.randn(dm, generator=g)
    dout = torch.randn(B, L, dm, generator=g)
    idx = _index(base, t, cu, L, mrd, dev)
    yd, Wd, bd = y.to(dev), W.to(dev), bias.to(dev)
    out = rd.restore_proj_fwd_indexed(yd, idx, B * D, D, L, Wd, bd)
    dy, dW = rd.restore_proj_bwd_indexed(dout.to(dev), yd, idx, B * D, D, L, Wd)
    torch.cuda.synchronize()
    # float64 composition with autograd
    y64 = y.double().requires_grad_(True)
    W64 = W.double().requires_grad_(True)
    b64 = bias.double().requires_grad_(True)

    class _Restore(torch.autograd.Function):
        @staticmethod
        def forward(ctx, yv):
            return torch.from_numpy(orc.restore_fwd(yv.detach().numpy(), t, cu, D, L))

        @staticmethod
        def backward(ctx, gz):
            return torch.from_numpy(orc.restore_bwd(gz.numpy(), t, cu, D, L))

    ref = F.linear(_Restore.apply(y64), W64, b64)
    ref.backward(dout.double())
    assert_close(out.cpu(), ref.detach().numpy(), RTOL, FLOOR, "out")
    if E:
        assert_close(dy.cpu(), y64.grad.numpy(), RTOL, FLOOR, "dy")
    assert_close(dW.cpu(), W64.grad.numpy(), RTOL, FLOOR, "dW")


def test_restore_proj_skips_and_matches_unfused(cuda_device):
    """dy / dW computed alone equal the joint call (the kernels are the
    same), and the op equals the unfused GPU composition restore ->
    F.linear within the fp32 bar."""
    dev = cuda_device
    B, D, L, dm = 2, 128, 640, 96
    base, ch, t, cu = _events(B, D, L, 0.1, seed=11)
    idx = _index(base, t, cu, L, 1, dev)
    g = torch.Generator().manual_seed(5)
    y = torch.randn(len(t), generator=g).to(dev)
    W = (torch.randn(dm, D, generator=g) / np.sqrt(D)).to(dev)
    dout = torch.randn(B, L, dm, generator=g).to(dev)
    dy, dW = rd.restore_proj_bwd_indexed(dout, y, idx, B * D, D, L, W)
    dy1, none1 = rd.restore_proj_bwd_indexed(dout, y, idx, B * D, D, L, W, need_dw=False)
    none2, dW1 = rd.restore_proj_bwd_indexed(dout, y, idx, B * D, D, L, W, need_dy=False)
    assert none1 is None and none2 is None
    assert torch.equal(dy, dy1) and torch.equal(dW, dW1)
    out = rd.restore_proj_fwd_indexed(y, idx, B * D, D, L, W)
    z = rd.restore_fwd_indexed(y, idx, B * D, D, L)
    ref = F.linear(z, W)
    assert_close(out.cpu(), ref.double().cpu().numpy(), RTOL, FLOOR, "out vs restore + linear")
