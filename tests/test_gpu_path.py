"""End-to-end parity of the event path (extract -> gather -> scan -> restore,
forward and backward) and of the Mamba block, on the GPU."""
import numpy as np
import pytest
import torch

from bc_mamba_amd import e_model
from bc_mamba_amd import extract_events_cuda as ee
from bc_mamba_amd import selective_scan_cuda as ssc
from bc_mamba_amd.selective_scan_interface import selective_scan_flat_ch_fn
from bc_mamba_amd.workloads import make_workload
from conftest import assert_close
from oracle import event_path as orc
from oracle import torch_path as tp

pytestmark = pytest.mark.gpu


def api_path(w, dev):
    """The reference composition through the drop-in API (autograd)."""
    x_conv = w.x_conv.to(dev).requires_grad_(True)
    params = [p.to(dev).requires_grad_(True) for p in (w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C, w.D_skip)]
    ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane.to(dev), w.threshold)
    u = e_model.GatherEventsFn.apply(x_conv, ch, t)
    y, x = selective_scan_flat_ch_fn(u, k, cu, int(ms), *params[:5], D=params[5], is_depthwise_bc=True)
    out = e_model.restore_dense_fn(y, t, cu, w.D, w.L)
    out.backward(w.dout.to(dev))
    return out.detach(), [x_conv.grad] + [p.grad for p in params], int(ch.numel())


def test_path_config0_matches_torch_formulation(cuda_device):
    w = make_workload(0)
    out, grads, E = api_path(w, cuda_device)
    d = lambda v: v.double()
    ref_out, ref_g, rE = tp.path_fwd_bwd(w.membrane, d(w.x_conv), d(w.dout), w.threshold, d(w.dt_idle),
                                          d(w.dt_active), d(w.A), d(w.W_B), d(w.W_C), d(w.D_skip))
    assert E == rE
    assert_close(out.cpu(), ref_out, 1e-4, 1e-6, "out")
    for name, g, r in zip(("x_conv", "dt_idle", "dt_active", "A", "W_B", "W_C", "D"), grads,
                          [ref_g[n] for n in ("x_conv", "dt_idle", "dt_active", "A", "W_B", "W_C", "D")]):
        assert_close(g.cpu(), r, 1e-4, 1e-6, name)


@pytest.mark.parametrize("expand", [1, 2])
def test_mamba_block_fused_matches_reference_composition(cuda_device, expand):
    torch.manual_seed(0)
    blk = e_model.Mamba(d_model=32, d_state=16, expand=expand, device=cuda_device, fused_event_path=True)
    torch.manual_seed(1)
    hs = (torch.rand(3, 300, 32, device=cuda_device) > 0.7).float()  # spike-like membrane
    outs, grads = [], []
    for fused in (True, False):
        blk.fused_event_path = fused
        blk.zero_grad()
        h = hs.clone().requires_grad_(True)
        o = blk(h)
        (o * torch.linspace(-1, 1, o.numel(), device=cuda_device).view_as(o)).sum().backward()
        outs.append(o.detach())
        grads.append({n: p.grad.detach().clone() for n, p in blk.named_parameters() if p.grad is not None})
    # the two paths differ in conv and scan rounding order: the fp32 parity bar
    assert_close(outs[0].cpu(), outs[1].cpu().numpy(), 1e-4, 1e-5, "block out")
    assert grads[0].keys() == grads[1].keys() and "W_BC" in grads[0] and "A_log" in grads[0]
    for n in grads[0]:
        assert_close(grads[0][n].cpu(), grads[1][n].cpu().numpy(), 1e-4, 1e-5, n)


def test_config1_full_size_properties(cuda_device):
    w = make_workload(1).to(cuda_device)
    ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane, w.threshold)
    E = ch.numel()
    assert E == int(w.membrane.sum().item())
    # gaps rebuild the event times inside each channel
    first = torch.ones(E, dtype=torch.bool, device=cuda_device)
    first[1:] = ch[1:] != ch[:-1]
    seg = torch.cumsum(first.long(), 0) - 1
    csum = torch.cumsum(k.long(), 0)
    base = torch.zeros(int(seg.max()) + 1, dtype=torch.long, device=cuda_device)
    base.index_copy_(0, seg[first], (csum - k.long())[first])
    assert torch.equal(csum - base[seg] - 1, t.long())
    # scan on a sample of channels against the oracle (channels are independent)
    u = ee.gather_events_fwd(w.x_conv, ch, t)[0]
    out, x = ssc.fwd_flat_ch(u, k, cu, int(ms), w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C, D=w.D_skip,
                             is_depthwise_bc=True)
    dout = torch.randn(E, device=cuda_device, generator=torch.Generator(device=cuda_device).manual_seed(3))
    gb = ssc.bwd_flat_ch(u, k, cu, int(ms), w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C, dout, x, D=w.D_skip,
                         is_depthwise_bc=True)
    cu_h = cu.cpu().numpy()
    b = 7
    sel = np.arange(b * w.D, b * w.D + 64)  # channels d = 0..63 of batch 7
    s, e = cu_h[sel[0]], cu_h[sel[-1] + 1]
    cu_s = (cu_h[sel[0]:sel[-1] + 2] - s).astype(np.int32)
    n = lambda v: v.detach().float().cpu().numpy()
    ms_s = int(np.diff(cu_s).max())
    P = lambda v: n(v)[:64]
    ref_out, ref_x = orc.scan_fwd(n(u)[s:e], n(k.float()).astype(np.int32)[s:e], cu_s, ms_s, P(w.dt_idle),
                                  P(w.dt_active), P(w.A), P(w.W_B), P(w.W_C), P(w.D_skip))
    assert_close(n(out)[s:e], ref_out, 1e-4, 1e-6, "out sample")
    assert_close(n(x)[sel], ref_x, 1e-4, 1e-6, "x sample")
    ref_g = orc.scan_bwd(n(u)[s:e], n(k.float()).astype(np.int32)[s:e], cu_s, ms_s, P(w.dt_idle), P(w.dt_active),
                         P(w.A), P(w.W_B), P(w.W_C), n(dout)[s:e], P(w.D_skip))
    assert_close(n(gb[0])[s:e], ref_g[0], 1e-4, 1e-6, "du sample")
    # parameter gradients are sums over the 32 batches: compare with the sum of per-batch oracle runs would be
    # costly; the ddt_active of dim d equals the sum over its channels of dΔ, checked through linearity:
    g2 = ssc.bwd_flat_ch(u, k, cu, int(ms), w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C, 2.0 * dout, x, D=w.D_skip,
                         is_depthwise_bc=True)
    for a, b2 in zip(gb, g2):
        assert_close(n(b2), 2.0 * n(a), 1e-5, 1e-6, "linearity")


def test_config4_model_fused_matches_reference_composition(cuda_device):
    """The config-4 model (lra_impl.py:1429-1615 composition, small sizes):
    a training step through every block's fused event path (HIP extraction,
    conv, scan, restore) matches the reference composition (nn.Conv1d,
    reference-order extraction and restore) in loss and every gradient."""
    from bc_mamba_amd.workloads import make_model_workload
    model, tokens, labels = make_model_workload(seed=3, B=2, L=200, device=cuda_device, d_model=32, n_layers=2)
    losses, grads = [], []
    for fused in (True, False):
        for blk in model.blocks:
            blk.core.fused_event_path = fused
        model.zero_grad()
        loss = torch.nn.functional.cross_entropy(model(tokens), labels)
        loss.backward()
        losses.append(float(loss))
        grads.append({n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None})
    assert np.isfinite(losses[0]) and losses[0] == pytest.approx(losses[1], rel=1e-5)
    assert grads[0].keys() == grads[1].keys() and len(grads[0]) > 10
    for n in grads[0]:
        assert_close(grads[0][n].cpu(), grads[1][n].cpu().numpy(), 1e-3, 1e-4, n)


def test_mamba_block_conv_at_events_matches_dense_conv(cuda_device):
    """The fused block with the conv evaluated at the events equals the
    fused block with the dense HIP conv: output and the scan / projection
    gradients bit for bit; the conv weight / bias gradients (summed in
    another order) and those behind in_proj (its GEMM sees dx in another
    layout) within the fp32 bar."""
    torch.manual_seed(0)
    blk = e_model.Mamba(d_model=32, d_state=16, expand=2, device=cuda_device)
    torch.manual_seed(1)
    hs = (torch.rand(3, 304, 32, device=cuda_device) > 0.7).float()
    outs, grads = [], []
    for at_events in (True, False):
        blk.conv_at_events = at_events
        blk.zero_grad()
        h = hs.clone().requires_grad_(True)
        o = blk(h)
        (o * torch.linspace(-1, 1, o.numel(), device=cuda_device).view_as(o)).sum().backward()
        outs.append(o.detach())
        grads.append({n: p.grad.detach().clone() for n, p in blk.named_parameters() if p.grad is not None})
        grads[-1]["input"] = h.grad.detach().clone()
    assert torch.equal(outs[0], outs[1])
    assert grads[0].keys() == grads[1].keys() and "conv1d.weight" in grads[0]
    for n in grads[0]:
        if n.startswith(("conv1d.", "in_proj.")) or n == "input":
            assert_close(grads[0][n].cpu(), grads[1][n].cpu().numpy(), 1e-4, 1e-5, n)
        else:
            assert torch.equal(grads[0][n], grads[1][n]), n


def test_split_k_projections_on_gpu(cuda_device):
    """The block's split-K projection gradients on the GPU (hipBLASLt batched
    products) agree with torch's plain products within fp32 rounding."""
    from bc_mamba_amd import projections as pj
    torch.manual_seed(0)
    M = 4 * pj.MIN_TOKENS
    x = torch.randn(4, M // 4, 256, device=cuda_device, requires_grad=True)
    w = torch.randn(128, 256, device=cuda_device, requires_grad=True)
    b = torch.randn(128, device=cuda_device, requires_grad=True)
    gy = torch.randn(4, M // 4, 128, device=cuda_device)
    pj.linear(x, w, b).backward(gy)
    x2, w2, b2 = (t.detach().clone().requires_grad_(True) for t in (x, w, b))
    torch.nn.functional.linear(x2, w2, b2).backward(gy)
    assert_close(w.grad.cpu(), w2.grad.cpu().numpy(), 1e-4, 1e-5, "dweight")
    assert_close(b.grad.cpu(), b2.grad.cpu().numpy(), 1e-4, 1e-5, "dbias")
    assert_close(x.grad.cpu(), x2.grad.cpu().numpy(), 1e-5, 1e-6, "dx")
    h = torch.randn(M, 256, device=cuda_device, requires_grad=True)
    wi = torch.randn(512, 256, device=cuda_device, requires_grad=True)
    g = torch.randn(512, M, device=cuda_device)
    pj.proj_tokens_last(wi, h).backward(g)
    h2, wi2 = h.detach().clone().requires_grad_(True), wi.detach().clone().requires_grad_(True)
    (wi2 @ h2.t()).backward(g)
    assert_close(wi.grad.cpu(), wi2.grad.cpu().numpy(), 1e-4, 1e-5, "in_proj dweight")
    assert_close(h.grad.cpu(), h2.grad.cpu().numpy(), 1e-5, 1e-6, "in_proj dh")
