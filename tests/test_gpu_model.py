"""The Mamba block (e_model.py:419-506) and the config-4 model on the GPU
against the float64 oracle composition (oracle/block.py: torch float64
dense parts around the numpy oracle's extraction, gather, scan and restore).

  block    the fused block (spike-bits head, conv at the events, indexed
           extraction / scan, the restore -> out_proj op in both modes,
           split-K projections) with expand 1 and 2: output and every
           parameter and input gradient at the fp32 bar (rtol 1e-4, floor
           1e-6 * max|ref|)
  config 4 one full-size training step (B50 L1024, d_model 256, d_inner
           512, 6 layers): finite loss and gradients, the loss of the
           reference composition (fused_event_path=False), every layer's
           block through both paths on the same input, and layer 0's output,
           input gradient and every parameter gradient against the oracle
           over the whole batch
"""
import numpy as np
import pytest
import torch

from bc_mamba_amd import e_model
from bc_mamba_amd.workloads import make_model_workload
from conftest import assert_close
from oracle import block as ob

pytestmark = pytest.mark.gpu


def _grads(blk, h):
    g = {n: p.grad.detach().float().cpu().clone() for n, p in blk.named_parameters() if p.grad is not None}
    g["input"] = h.grad.detach().float().cpu().clone()
    return g


@pytest.mark.parametrize("expand,out_proj", [(1, True), (2, True), (2, "mfma")])
def test_mamba_block_matches_oracle(cuda_device, expand, out_proj):
    """The fused block behind its spike head, against the float64 oracle
    composition on the same parameters: same spikes, then output and every
    gradient (in_proj, conv weight / bias, W_BC, A_log, D, the two dt
    levels, out_proj, prob_head, and the head's input). out_proj: the
    restore -> out_proj op's mode (hipBLASLt products around the fused dy
    kernel, or all three of this package's matrix-core kernels)."""
    torch.manual_seed(0)
    blk = e_model.Mamba(d_model=32, d_state=16, expand=expand, device=cuda_device, fused_out_proj=out_proj)
    with torch.no_grad():  # non-trivial values where the initialisation is flat
        blk.W_BC.normal_(0.0, 0.3)
        blk.D.uniform_(0.5, 1.5)
    gen = torch.Generator().manual_seed(1)
    v = torch.randn(3, 300, 32, generator=gen) * 2.0
    gout = torch.randn(3, 300, 32, generator=gen)
    # GPU: spike head (one kernel: s and its event bits), then the block
    vg = v.to(cuda_device).requires_grad_(True)
    s = blk.to_spike(vg)
    assert getattr(s, "_bcm_event_bits", None) is not None  # the bits path runs
    out = blk(s)
    out.backward(gout.to(cuda_device))
    got = _grads(blk, vg)
    # oracle
    p = ob.params_of(blk)
    v64 = v.double().requires_grad_(True)
    s64, prob = ob.spike_head(blk, v64, p)
    assert torch.equal(s.detach().cpu() > 0.5, s64.detach() > 0.5)  # same spikes in fp32 and fp64
    out64, p = ob.mamba_forward(blk, s64, p=p)
    out64.backward(gout.double())
    ref = {n: q.grad for n, q in p.items() if q.grad is not None}
    ref["input"] = v64.grad
    assert_close(out.detach().cpu(), out64.detach().numpy(), 1e-4, 1e-6, "block out")
    assert got.keys() == ref.keys() and len(got) >= 11, (sorted(got), sorted(ref))
    for name in ref:
        assert_close(got[name], ref[name].numpy(), 1e-4, 1e-6, name)


def test_config4_full_size_model_step(cuda_device):
    """Config 4 at full size (B50 L1024 d_model 256 d_inner 512 N16, six
    layers, byte tokens, random init): one training step."""
    dev = cuda_device
    model, tokens, labels = make_model_workload(device=dev)
    captured = []

    def grab(mod, args):
        s = args[0]
        captured.append((s.detach(), getattr(s, "_bcm_event_bits", None)))

    hooks = [blk.core.register_forward_pre_hook(grab) for blk in model.blocks]
    loss = torch.nn.functional.cross_entropy(model(tokens), labels)
    loss.backward()
    for h in hooks:
        h.remove()
    assert len(captured) == len(model.blocks) == 6
    assert np.isfinite(float(loss.detach()))
    assert all(torch.isfinite(p.grad).all() for p in model.parameters() if p.grad is not None)
    assert all(c[1] is not None for c in captured)  # every block took its input's spike bits
    # the reference composition (nn.Conv1d, reference-order extraction,
    # restore and projections) over the whole model: the same loss
    for blk in model.blocks:
        blk.core.fused_event_path = False
    model.zero_grad()
    with torch.no_grad():
        loss_ref = torch.nn.functional.cross_entropy(model(tokens), labels)
    assert abs(float(loss.detach()) - float(loss_ref)) <= 1e-4 * abs(float(loss_ref))
    # every layer's block through both paths on the same input spikes
    gen = torch.Generator().manual_seed(7)
    for i, blk in enumerate(model.blocks):
        core = blk.core
        s, bits = captured[i]
        gout = torch.randn(s.shape, generator=gen).to(dev)
        res = []
        for fused in (True, False):
            core.fused_event_path = fused
            core.zero_grad()
            h = s.clone().requires_grad_(True)
            if fused:
                h._bcm_event_bits = (bits[0], bits[1], h._version)
            o = core(h)
            o.backward(gout)
            res.append((o.detach().float().cpu(), _grads(core, h)))
        print(f"layer {i}: fused vs reference composition", flush=True)
        # two fp32 implementations (HIP conv at the events / MIOpen conv,
        # split-K / plain projections, scan and restore in different
        # orders): each side's rounding enters, so the floor is 1e-5
        assert_close(res[0][0], res[1][0].numpy(), 1e-4, 1e-5, f"layer {i} out")
        for name in res[1][1]:
            assert_close(res[0][1][name], res[1][1][name].numpy(), 1e-4, 1e-5, f"layer {i} {name}")
        core.fused_event_path = True
    # layer 0 against the float64 oracle over the whole batch (B = 50):
    # output, input gradient and every parameter gradient
    core = model.blocks[0].core
    s, bits = captured[0]
    gout = torch.randn(s.shape, generator=gen)
    core.zero_grad()
    h = s.clone().requires_grad_(True)
    h._bcm_event_bits = (bits[0], bits[1], h._version)
    o = core(h)
    o.backward(gout.to(dev))
    got = _grads(core, h)
    h64 = s.double().cpu().requires_grad_(True)
    out64, p64 = ob.mamba_forward(core, h64)
    out64.backward(gout.double())
    ref = {n: q.grad for n, q in p64.items() if q.grad is not None}
    ref["input"] = h64.grad
    print("layer 0 against the oracle, B = 50", flush=True)
    assert_close(o.detach().cpu(), out64.detach().numpy(), 1e-4, 1e-6, "layer 0 out")
    assert got.keys() == ref.keys() and len(got) >= 10, (sorted(got), sorted(ref))
    for name in ref:
        r = ref[name].numpy()
        err = float(np.max(np.abs(got[name].numpy() - r) / (1e-4 * np.abs(r) + 1e-6 * np.abs(r).max() + 1e-300)))
        print(f"  {name}: error / fp32 bar = {err:.3f}", flush=True)
        assert_close(got[name], r, 1e-4, 1e-6, f"layer 0 {name}")
