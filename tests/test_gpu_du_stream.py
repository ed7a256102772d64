"""The fused step without the du stream (keep_du=False: the scan backward
writes dx's rows itself and stores no separate du, as the model's backward
does) against the step with it: dx, the parameter gradients and every
forward output are bit-equal, and dx holds du at the events."""
import pytest
import torch

from bc_mamba_amd import _native as nat
from bc_mamba_amd.fused_step import FusedStep
from bc_mamba_amd.workloads import make_workload

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg,B", [(1, 16), (2, 16)])
def test_step_without_du_stream_matches(cuda_device, cfg, B):
    print(f"du stream: config {cfg} B={B}", flush=True)
    w = make_workload(cfg, B=B).to(cuda_device)
    full = FusedStep(w, cuda_device)
    full.step()
    lean = FusedStep(w, cuda_device, keep_du=False)
    lean.du_buf.fill_(float("nan"))  # nothing may read or keep the unused buffer's contents
    lean.step()
    torch.cuda.synchronize()
    assert full.args.du is not None and lean.args.du is None  # the one-kernel backward applies at these shapes
    assert torch.isnan(lean.du_buf[:lean.E]).all()  # no du stored
    for name in ("y", "dense", "dy_restore", "dx"):
        assert torch.equal(getattr(full, name), getattr(lean, name)), name
    for i, (a, b) in enumerate(zip(full.grads, lean.grads)):
        assert torch.equal(a, b), f"grad {i}"
    # dx carries du at the events: times rebuilt from the gaps k within each
    # channel (k = t + 1 for a channel's first event, else the gap)
    cu = full.cu.long()
    ch = torch.repeat_interleave(torch.arange(full.NC, device=cuda_device), cu[1:] - cu[:-1])
    k = full.k.long()
    csum = torch.cumsum(k, 0)
    start = cu[ch]
    t = csum - (csum[start] - k[start]) - 1
    assert torch.equal(full.dx.view(full.NC, w.L)[ch, t], full.du)


def test_query_matches_the_path_taken(cuda_device):
    w = make_workload(1, B=16).to(cuda_device)
    st = FusedStep(w, cuda_device, keep_du=False)
    st.step()
    assert nat.lib().bcm_scan_bwd_rows_fused(st.args, st.rows) == 1
