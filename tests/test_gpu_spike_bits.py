"""GPU parity of the fused straight-through spike head (bcm_spike_bits, f1
of the path's next steps): s bit-identical to the reference's
(p >= thr) + p - p (e_model.py:233-254), the event bitmask equal to the
bits of the transposed spikes, the extraction fed from those bits equal to
the one fed from the membrane, and the config-4 model identical with and
without the fused head."""
import numpy as np
import pytest
import torch

from bc_mamba_amd import extract_events_cuda as ee
from oracle import event_path as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,L,Dm,thr,dtype", [
    (2, 64, 64, 0.5, torch.float32),
    (3, 1000, 96, 0.5, torch.float32),     # partial tile and a partial channel group
    (2, 300, 40, 0.3, torch.float32),
    (2, 257, 130, 0.2999, torch.bfloat16),  # threshold not representable in bf16
    (1, 128, 64, 0.7, torch.float16),
])
def test_spike_bits_match_ste_and_mask(cuda_device, B, L, Dm, thr, dtype):
    print(f"spike bits case B={B} L={L} Dm={Dm} thr={thr} {dtype}", flush=True)
    g = torch.Generator().manual_seed(L + Dm)
    p = torch.rand(B, L, Dm, generator=g).to(dtype).to(cuda_device)
    s, bitmask = ee.spike_bits(p, thr)
    ref = (p >= thr).to(p.dtype) + p - p  # the reference's STE value
    assert torch.equal(s, ref)
    hard = (p >= thr).permute(0, 2, 1).reshape(B * Dm, L).cpu().numpy()
    nw = (L + 31) // 32
    words = bitmask[:, :nw].cpu().numpy().view(np.uint32)
    bits = np.unpackbits(words.view(np.uint8), bitorder="little").reshape(B * Dm, nw * 32)[:, :L]
    assert np.array_equal(bits.astype(bool), hard)
    if dtype == torch.float32:  # the CPU oracle of the spike head
        os_, obits = orc.spike_ste(p.cpu().numpy(), thr)
        assert np.array_equal(s.cpu().numpy(), os_) and np.array_equal(bits.astype(bool), obits)


@pytest.mark.parametrize("expand", [1, 2])
def test_extraction_from_bits_matches_membrane(cuda_device, expand):
    B, L, Dm = 3, 700, 48
    g = torch.Generator().manual_seed(expand)
    p = torch.rand(B, L, Dm, generator=g).to(cuda_device)
    x = torch.randn(B, Dm * expand, L, generator=g).to(cuda_device)
    s, bitmask = ee.spike_bits(p, 0.7)
    mem = s.permute(0, 2, 1).contiguous()  # the reference's transposed membrane
    ref = ee.extract_events_indexed(mem, 0.5, expand, x, positions=True)
    got = ee.extract_events_indexed(None, 0.5, expand, x, positions=True, bits=(bitmask, (B, Dm, L)))
    for i in (0, 1, 2, 3, 5):
        assert torch.equal(ref[i], got[i]), i
    assert ref[4] == got[4]
    nw = (L + 31) // 32
    assert torch.equal(ref[6][0][:, :nw], got[6][0][:, :nw]) and torch.equal(ref[6][1], got[6][1])


def test_model_with_fused_spike_head_is_identical(cuda_device):
    from bc_mamba_amd.workloads import make_model_workload
    model, tokens, labels = make_model_workload(seed=5, B=2, L=256, device=cuda_device, d_model=64, n_layers=2)
    samplers = [m for m in model.modules() if m.__class__.__name__ == "SpikeSamplerSurrogate"]
    assert samplers
    losses, grads = [], []
    for fused in (True, False):
        for m in samplers:
            m.fused_bits = fused
        model.zero_grad()
        loss = torch.nn.functional.cross_entropy(model(tokens), labels)
        loss.backward()
        losses.append(loss.detach())
        grads.append({n: q.grad.detach().clone() for n, q in model.named_parameters() if q.grad is not None})
    assert torch.equal(losses[0], losses[1])
    assert grads[0].keys() == grads[1].keys()
    for n in grads[0]:
        assert torch.equal(grads[0][n], grads[1][n]), n
