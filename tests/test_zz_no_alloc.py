"""The allocation-free restore backward (bcm_restore_bwd_noalloc) against the
workspace entry point (bcm_restore_bwd) through the C ABI: the same kernels,
so dy must be bit-identical, on two calls in a row (the second smaller, so it
runs on scratch the first one left behind), plus the oracle at rtol 1e-4."""
import pytest
import torch

from bc_mamba_amd import _native as nat
from bc_mamba_amd import extract_events_cuda as ee
from conftest import assert_close
from oracle import event_path as orc

pytestmark = pytest.mark.gpu


def _case(B, D, L, p, seed, dev, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    mem = (torch.rand(B, D, L, generator=g) < p).float()
    dout = torch.randn(B, L, D, generator=g).to(dtype)
    ch, t, k, cu, ms, _, (bitmask, tile_start, mrd) = ee.extract_events_indexed(mem.to(dev), 0.5, positions=True)
    return dict(B=B, D=D, L=L, dout=dout.to(dev), t=t, cu=cu, bitmask=bitmask, tile_start=tile_start, mrd=mrd)


def _restore_bwd(c, noalloc):
    dev = c["dout"].device
    E = int(c["t"].numel())
    NC = c["B"] * c["D"]
    dy = torch.full((E,), float("nan"), dtype=torch.float32, device=dev)
    P, s = nat.ptr, nat.stream_of(c["dout"])
    args = (P(c["dout"]), nat.dtype_code(c["dout"].dtype), P(c["bitmask"]), int(c["mrd"]), P(c["tile_start"]), NC,
            c["D"], c["L"], P(dy), E)
    if noalloc:
        nat.call("bcm_restore_bwd_noalloc", *args, s)
    else:
        ws = torch.empty(nat.lib().bcm_restore_bwd_workspace_bytes(NC, c["L"]) // 4, dtype=torch.float32, device=dev)
        nat.call("bcm_restore_bwd", *args, P(ws), 4 * ws.numel(), s)
    return dy


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_restore_bwd_noalloc_matches_workspace_entry(cuda_device, dtype):
    # config-1 shape first, then a smaller one on the scratch it leaves behind
    for (B, D, L, p, seed) in ((32, 256, 2048, 0.15, 0), (3, 64, 700, 0.3, 1)):
        print(f"noalloc case B={B} D={D} L={L} p={p} {dtype}", flush=True)
        c = _case(B, D, L, p, seed, cuda_device, dtype)
        ref = _restore_bwd(c, noalloc=False)
        got = _restore_bwd(c, noalloc=True)
        torch.cuda.synchronize()
        assert not torch.isnan(got).any()
        assert torch.equal(got, ref)
        if B * D <= 256:  # the oracle at a size it finishes in well under a second
            t, cu = c["t"].cpu().numpy(), c["cu"].cpu().numpy()
            want = orc.restore_bwd(c["dout"].float().cpu().numpy(), t, cu, D, L)
            assert_close(got.cpu().numpy(), want, 1e-4 if dtype == torch.float32 else 2e-2, 1e-6, "dy")
