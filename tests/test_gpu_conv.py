"""GPU parity of the causal depthwise conv1d + SiLU (the producer of
x_conv, e_model.py:442-451) against the CPU oracle: fp32 within rtol 1e-4,
bf16 within 2e-2; dw / dbias reduced deterministically."""
import numpy as np
import pytest
import torch

from bc_mamba_amd.causal_conv1d import causal_conv1d_fn
from conftest import assert_close
from oracle import event_path as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,D,L,K,act,bias", [
    (2, 8, 64, 4, "silu", True),
    (3, 5, 37, 4, "silu", True),      # L not a multiple of the 4 steps per thread
    (2, 4, 1025, 4, None, False),     # no activation, no bias, a 1025-step row
    (1, 3, 50, 1, "silu", True),
    (2, 6, 300, 7, "swish", True),
    (2, 6, 300, 8, "silu", False),
    (4, 512, 1024, 4, "silu", True),  # config-4 layer shape per batch row
])
def test_conv1d_fp32(cuda_device, B, D, L, K, act, bias):
    print(f"conv case B={B} D={D} L={L} K={K} act={act} bias={bias}", flush=True)
    g = torch.Generator().manual_seed(B * 1000 + L + K)
    x = torch.randn(B, D, L, generator=g)
    w = torch.randn(D, K, generator=g) / K
    b = torch.randn(D, generator=g) if bias else None
    dout = torch.randn(B, D, L, generator=g)
    dev = cuda_device
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    bd = b.to(dev).requires_grad_(True) if bias else None
    y = causal_conv1d_fn(xd, wd, bd, activation=act)
    y.backward(dout.to(dev))
    silu = act is not None
    ref = orc.conv1d_fwd(x.numpy(), w.numpy(), b.numpy() if bias else None, silu)
    dx, dw, db = orc.conv1d_bwd(x.numpy(), w.numpy(), b.numpy() if bias else None, dout.numpy(), silu)
    assert_close(y.detach().cpu(), ref, 1e-4, 1e-5, "out")
    assert_close(xd.grad.cpu(), dx, 1e-4, 1e-5, "dx")
    assert_close(wd.grad.cpu(), dw, 1e-4, 1e-5, "dw")
    if bias:
        assert_close(bd.grad.cpu(), db, 1e-4, 1e-5, "dbias")


def test_conv1d_bf16_and_deterministic(cuda_device):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 16, 500, generator=g).to(torch.bfloat16)
    w = torch.randn(16, 4, generator=g) / 4
    b = torch.randn(16, generator=g)
    dout = torch.randn(3, 16, 500, generator=g).to(torch.bfloat16)
    dev = cuda_device
    outs = []
    for _ in range(2):
        xd, wd, bd = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
        y = causal_conv1d_fn(xd, wd, bd, activation="silu")
        y.backward(dout.to(dev))
        outs.append((y.detach(), xd.grad, wd.grad, bd.grad))
    assert all(torch.equal(p, q) for p, q in zip(*outs))
    y, dxg, dwg, dbg = outs[0]
    assert y.dtype == torch.bfloat16 and dxg.dtype == torch.bfloat16
    xf, df = x.float().numpy(), dout.float().numpy()
    assert_close(y.float().cpu(), orc.conv1d_fwd(xf, w.numpy(), b.numpy()), 2e-2, 2e-3, "out")
    dx, dw, db = orc.conv1d_bwd(xf, w.numpy(), b.numpy(), df)
    assert_close(dxg.float().cpu(), dx, 2e-2, 2e-3, "dx")
    assert_close(dwg.cpu(), dw, 2e-2, 2e-3, "dw")
    assert_close(dbg.cpu(), db, 2e-2, 2e-3, "dbias")
