"""GPU parity of stage 3 (zero-order-hold restore fwd / bwd) against the CPU
oracle (the reference's upper_bound search semantics)."""
import numpy as np
import pytest
import torch

from bc_mamba_amd import restore_dense_cuda_nodecay as rd
from conftest import assert_close
from oracle import event_path as orc

pytestmark = pytest.mark.gpu


def _events(B, D, L, p, seed, empty_every=0):
    g = torch.Generator().manual_seed(seed)
    mem = (torch.rand(B, D, L, generator=g) < p).float()
    if empty_every:
        mem.view(B * D, L)[::empty_every] = 0.0
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem.numpy(), 0.5)
    return ch, t, cu


CASES = [  # B, D, L, density
    (2, 256, 2048, 0.15),  # config-1 channel layout, fewer batches
    (2, 100, 500, 0.3),    # D not a multiple of 64
    (3, 7, 65, 0.5),       # ragged last tile
    (1, 3, 1, 0.9),
    (1, 2, 6000, 0.9),     # > 4095 events per channel (beyond the reference's exact range)
    (2, 64, 300, 0.02),
    (1, 64, 256, 0.6),     # > 1024 events per 64-channel tile: the backward's direct-store path
]


@pytest.mark.parametrize("B,D,L,p", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_restore_fwd_bwd(cuda_device, B, D, L, p, dtype):
    """16-bit values with an even D take the two-channels-per-lane forward
    (an odd D the one-channel form); every value is a copy: bit-exact."""
    print(f"restore case B={B} D={D} L={L} p={p} {dtype}", flush=True)
    ch, t, cu = _events(B, D, L, p, seed=L + D, empty_every=5)
    g = torch.Generator().manual_seed(1)
    y = torch.randn(len(t), generator=g).to(dtype)
    dout = torch.randn(B, L, D, generator=g).to(dtype)
    t_d, cu_d = torch.from_numpy(t).to(cuda_device), torch.from_numpy(cu).to(cuda_device)
    out = rd.restore_dense_fwd(y.to(cuda_device), t_d, cu_d, D, L)
    assert out.dtype == dtype and tuple(out.shape) == (B, L, D)
    ref = orc.restore_fwd(y.float().numpy(), t, cu, D, L)
    assert np.array_equal(out.float().cpu().numpy(), ref.astype(np.float32))  # a copy: bit-exact
    dy = rd.restore_dense_bwd(dout.to(cuda_device), t_d, cu_d, D, L)
    assert dy.dtype == torch.float32 and dy.numel() == len(t)
    assert_close(dy.cpu(), orc.restore_bwd(dout.float().numpy(), t, cu, D, L), 1e-5, 1e-6, "dy")


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
def test_restore_fp32_to_half_out(cuda_device, out_dtype):
    B, D, L = 2, 70, 300
    ch, t, cu = _events(B, D, L, 0.2, seed=3)
    y = torch.randn(len(t))
    out = rd.restore_dense_fwd(y.to(cuda_device), torch.from_numpy(t).to(cuda_device),
                               torch.from_numpy(cu).to(cuda_device), D, L, out_dtype)
    ref = torch.from_numpy(orc.restore_fwd(y.numpy(), t, cu, D, L)).float().to(out_dtype)
    assert out.dtype == out_dtype and torch.equal(out.cpu(), ref)


def test_restore_no_events(cuda_device):
    B, D, L = 2, 3, 100
    t = torch.zeros(0, dtype=torch.int32, device=cuda_device)
    cu = torch.zeros(B * D + 1, dtype=torch.int32, device=cuda_device)
    out = rd.restore_dense_fwd(torch.zeros(0, device=cuda_device), t, cu, D, L)
    assert torch.count_nonzero(out) == 0 and tuple(out.shape) == (B, L, D)
    dy = rd.restore_dense_bwd(torch.randn(B, L, D, device=cuda_device), t, cu, D, L)
    assert dy.numel() == 0


def test_restore_adjoint_full_config1_shape(cuda_device):
    # size-independent property at the headline shape: <R y, g> == <y, R^T g>
    B, D, L = 32, 256, 2048
    g = torch.Generator(device=cuda_device).manual_seed(5)
    mem = (torch.rand(B, D, L, device=cuda_device, generator=g) < 0.15)
    from bc_mamba_amd import extract_events_cuda as ee
    ch, t, k, cu, counts, ms = ee.extract_base_events(mem.float(), 0.5)
    y = torch.randn(t.numel(), device=cuda_device, generator=g, dtype=torch.float64).float()
    gd = torch.randn(B, L, D, device=cuda_device, generator=g)
    out = rd.restore_dense_fwd(y, t, cu, D, L)
    dy = rd.restore_dense_bwd(gd, t, cu, D, L)
    lhs = (out.double() * gd.double()).sum().item()
    rhs = (y.double() * dy.double()).sum().item()
    assert lhs == pytest.approx(rhs, rel=1e-5)
    # every event value appears at its own time step
    b, d = ch.long() // D, ch.long() % D
    assert torch.equal(out[b, t.long(), d], y)
