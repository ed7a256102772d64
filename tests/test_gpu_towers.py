"""Config 3's two-tower encoding (the reference runs the towers as two
B = 32 calls, lra_impl.py:1685-1688): the fused step over two half-batch
calls against one call over the whole batch. Channels are independent, so
with the state-lane scans (whose per-channel arithmetic does not depend on
the other channels) every per-channel output is bit-equal; the parameter
gradients are the sum of the two calls' within the fp32 bar."""
import pytest
import torch

from bc_mamba_amd import _native as nat
from bc_mamba_amd.fused_step import FusedStep
from bc_mamba_amd.workloads import Workload, make_workload
from conftest import assert_close

pytestmark = pytest.mark.gpu


def _half(w, sl):
    f = {k: getattr(w, k) for k in w.__dataclass_fields__}
    f["B"] = sl.stop - sl.start
    for k in ("membrane", "x_conv", "dout"):
        f[k] = getattr(w, k)[sl].contiguous()
    return Workload(**f)


@pytest.mark.parametrize("restore_bwd", ["chained", "two_pass"])
def test_two_tower_calls_match_one_call(cuda_device, restore_bwd):
    print(f"towers: config 3 law at B8 D16 L1000 N64, restore bwd {restore_bwd}", flush=True)
    w = make_workload(3, B=8, D=16, L=1000).to(cuda_device)
    prev = nat.set_scan_family("lanes")
    try:
        one = FusedStep(w, cuda_device, restore_bwd=restore_bwd)
        one.step()
        parts = [FusedStep(_half(w, sl), cuda_device, restore_bwd=restore_bwd) for sl in (slice(0, 4), slice(4, 8))]
        for p in parts:
            p.step()
        torch.cuda.synchronize()
    finally:
        nat.set_scan_family(prev)
    assert one.E == sum(p.E for p in parts) and one.E > 0
    for name in ("k", "u", "y", "dy_restore", "du"):
        got = torch.cat([getattr(p, name) for p in parts])
        assert torch.equal(got, getattr(one, name)), name
    for name in ("dense", "dx"):
        got = torch.cat([getattr(p, name) for p in parts])
        assert torch.equal(got, getattr(one, name)), name
    for i, (g1, g2, g) in enumerate(zip(parts[0].grads, parts[1].grads, one.grads)):
        assert_close((g1 + g2).cpu(), g.cpu().numpy(), 1e-5, 1e-6, f"grad {i}")
