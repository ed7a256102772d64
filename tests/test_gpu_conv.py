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
    assert_close(y.detach().cpu(), ref, 1e-4, 1e-6, "out")
    assert_close(xd.grad.cpu(), dx, 1e-4, 1e-6, "dx")
    assert_close(wd.grad.cpu(), dw, 1e-4, 1e-6, "dw")
    if bias:
        assert_close(bd.grad.cpu(), db, 1e-4, 1e-6, "dbias")


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


# ---- the conv evaluated at the events (fill) and its backward from du ----
from bc_mamba_amd import extract_events_cuda as ee  # noqa: E402
from bc_mamba_amd.causal_conv1d import conv1d_bwd_events  # noqa: E402


def _in_proj_layout(x):
    """x [B, D, L] laid out as the block's in_proj output: a [D, B*L] matrix
    viewed as [B, D, L] (row (b, d) at d*B*L + b*L; rows contiguous)."""
    B, D, L = x.shape
    return x.permute(1, 0, 2).contiguous().view(D, B * L).view(D, B, L).permute(1, 0, 2)


@pytest.mark.parametrize("B,Dm,expand,L,K,silu,bias,dtype,strided", [
    (2, 8, 1, 256, 4, True, True, torch.float32, False),
    (3, 4, 2, 300, 4, True, True, torch.float32, True),     # in_proj layout, expanded channels
    (2, 4, 2, 1100, 3, True, False, torch.float32, True),   # width 3 (any-width form), two 1024-step windows
    (2, 6, 1, 64, 8, False, True, torch.float32, False),    # plain conv, width 8
    (2, 8, 2, 512, 4, True, True, torch.bfloat16, True),
    (2, 8, 1, 200, 4, True, True, torch.float16, False),
])
def test_conv_at_events_matches_dense_conv_then_gather(cuda_device, B, Dm, expand, L, K, silu, bias, dtype, strided):
    """x_events of the fill with conv (bcm_extract_fill_blocks_conv) equal
    bit for bit the dense conv followed by the gather; the backward from du
    (bcm_causal_conv1d_bwd_events) gives the dense path's dx bit for bit and
    its dweight / dbias within 1e-5 (fp32 sums in another order)."""
    print(f"conv-at-events case B={B} Dm={Dm} x{expand} L={L} K={K} silu={silu} {dtype} strided={strided}",
          flush=True)
    dev = cuda_device
    D = Dm * expand
    g = torch.Generator().manual_seed(L + K + B)
    mem = (torch.rand(B, Dm, L, generator=g) < 0.2).float().to(dev)
    x = torch.randn(B, D, L, generator=g).to(dtype).to(dev)
    if strided:
        x = _in_proj_layout(x)
        assert not x.is_contiguous() and x.stride(2) == 1
    w = (torch.randn(D, K, generator=g) / K).to(dev)
    b = torch.randn(D, generator=g).to(dev) if bias else None
    # dense reference: conv, then the fused extraction's gather
    xc = causal_conv1d_fn(x.contiguous(), w, b, activation="silu" if silu else None)
    _, _, k1, cu1, ms1, xe_ref, idx = ee.extract_events_indexed(mem, 0.5, expand, xc, positions=False)
    _, _, k2, cu2, ms2, xe, idx2 = ee.extract_events_indexed(mem, 0.5, expand, x, positions=False,
                                                            conv=(w, b, silu))
    assert torch.equal(k1, k2) and torch.equal(cu1, cu2) and ms1 == ms2
    nw = (L + 31) // 32  # bitmask rows are padded to 1024 steps; the padding words are not written
    assert torch.equal(idx[0][:, :nw], idx2[0][:, :nw]) and torch.equal(idx[1], idx2[1])
    assert xe.dtype == dtype and torch.equal(xe, xe_ref)
    # and against the CPU oracle: conv + SiLU evaluated at the oracle's events
    rtol, atol = (1e-4, 1e-6) if dtype == torch.float32 else (2e-2, 2e-3)
    och, ot, ok_, ocu, _, _ = orc.extract_base_events(mem.cpu().numpy(), 0.5)
    och, ot = orc.expand_base_events(och, ot, ok_, ocu, B, Dm, expand)[:2]
    xf = x.float().contiguous().cpu().numpy().reshape(B * D, L)
    assert_close(xe.float().cpu(), orc.conv_at_events(xf, w.cpu().numpy(), b.cpu().numpy() if bias else None,
                                                      och, ot, silu), rtol, atol, "x_events vs oracle")
    # backward: du at the events -> dense dx_conv -> dense conv backward
    du = torch.randn(xe.numel(), generator=g).to(dtype).to(dev)
    dxc = torch.empty(B * D, L, dtype=dtype, device=dev)
    ee._nat.call("bcm_gather_bwd_rows", du.data_ptr(), ee._nat.dtype_code(dtype), idx[0].data_ptr(), expand,
                 idx[1].data_ptr(), B * D, L, dxc.data_ptr(), ee._nat.stream_of(du))
    xr = x.contiguous().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    br = b.clone().requires_grad_(True) if bias else None
    causal_conv1d_fn(xr, wr, br, activation="silu" if silu else None).backward(dxc.view(B, D, L))
    dx, dw, db = conv1d_bwd_events(x, w, b, silu, du, idx2)
    torch.cuda.synchronize()
    assert dx.stride() == x.stride()
    assert torch.equal(dx, xr.grad)
    assert_close(dw.cpu(), wr.grad.cpu().numpy(), 1e-5, 1e-6, "dweight")
    if bias:
        assert_close(db.cpu(), br.grad.cpu().numpy(), 1e-5, 1e-6, "dbias")
    odx, odw, odb = orc.conv_bwd_events(xf.reshape(B, D, L), w.cpu().numpy(), b.cpu().numpy() if bias else None,
                                        du.float().cpu().numpy(), och, ot, silu)
    assert_close(dx.float().contiguous().cpu(), odx, rtol, atol, "dx vs oracle")
    assert_close(dw.cpu(), odw, rtol, atol, "dweight vs oracle")
    if bias:
        assert_close(db.cpu(), odb, rtol, atol, "dbias vs oracle")
