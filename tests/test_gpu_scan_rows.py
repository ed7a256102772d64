"""GPU parity of bcm_scan_bwd_rows, the model path's scan backward with the
gather backward folded in: du and every parameter gradient bit-identical
to bcm_scan_bwd, and dx [n_channels, L] bit-identical to the gather
backward of du (du at each channel's events, 0 elsewhere: the oracle's
scatter, extract_events_cuda.cu:717-754). Shapes cover the one-kernel form
(single-pass 16-lane shapes, L % 4 == 0, a partial last 64-step tile) and
the two-step form (multi-pass channels, z, L % 4 != 0), fp32 and 16-bit
inputs, empty channels and expanded channels that share mask rows."""
import numpy as np
import pytest
import torch

from bc_mamba_amd import restore_dense_cuda_nodecay as rdc
from bc_mamba_amd import selective_scan_cuda as ssc
from test_gpu_scan import _case

# every case under both dstate-16 kernel families (other dstates: the same kernel twice)
pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("scan_kernel")]

CASES = [  # B, D, L, density, N, dtype, with_z, p_short  (one kernel unless noted)
    (2, 8, 100, 0.5, 16, torch.float32, False, None),    # one 64-step tile and a partial one
    (2, 8, 448, 0.5, 16, torch.float32, False, None),
    (4, 16, 2048, 0.15, 16, torch.float32, False, None),  # config-1 shape class (16 x 24 items)
    (4, 16, 2048, 0.15, 16, torch.bfloat16, False, None),
    (2, 8, 1024, 0.3, 16, torch.float16, False, None),
    (2, 8, 230, 0.5, 16, torch.float32, False, None),    # L % 4 != 0: two steps
    (2, 8, 448, 0.5, 16, torch.float32, True, None),     # z: two steps
    (2, 8, 1200, 0.6, 16, torch.float32, False, 0.02),   # multi-pass channels: two steps
    (96, 2, 300, 0.5, 16, torch.float32, False, None),   # 96 channels per model channel: split workgroups
]


def _index(c, n_ch, L, dev, expand):
    """Event index of the case's channels; with expand > 1 consecutive
    channels share events and the bitmask keeps one row per group."""
    ts = torch.from_numpy(np.ascontiguousarray(c["t"], dtype=np.int32)).to(dev)
    cu = torch.from_numpy(np.ascontiguousarray(c["cu"], dtype=np.int32)).to(dev)
    bitmask, tile_start = rdc.build_event_index(ts, cu, L)
    if expand > 1:
        bitmask = bitmask[::expand].contiguous()
    return bitmask, tile_start


def _expanded_case(B, D, L, p, N, dtype, seed, with_z, p_short, expand):
    c = _case(B, D, L, p, N, dtype, seed, with_z=with_z, p_short=p_short, empty_every=5)
    if expand == 1:
        return c
    # channel ch repeats the events of channel expand * (ch // expand)
    cu = c["cu"]
    NC = len(cu) - 1
    lens = np.diff(cu)
    src = (np.arange(NC) // expand) * expand
    new_lens = lens[src]
    new_cu = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
    k = np.concatenate([c["k"][cu[s]:cu[s + 1]] for s in src]).astype(np.int32)
    t = np.concatenate([c["t"][cu[s]:cu[s + 1]] for s in src]).astype(np.int32)
    E = int(new_cu[-1])
    g = torch.Generator().manual_seed(seed + 1)
    c.update(k=k, t=t, cu=new_cu, ms=int(new_lens.max()) if NC else 0,
             u=torch.randn(E, generator=g).to(dtype), dout=torch.randn(E, generator=g).to(dtype),
             z=torch.randn(E, generator=g).to(dtype) if with_z else None)
    return c


@pytest.mark.parametrize("B,D,L,p,N,dtype,with_z,ps", CASES)
@pytest.mark.parametrize("expand,use_acc", [(1, False), (2, False), (1, True)])
def test_scan_bwd_rows_matches_scan_then_gather(cuda_device, B, D, L, p, N, dtype, with_z, ps, expand, use_acc):
    """bcm_scan_bwd_rows equals bcm_scan_bwd followed by the gather backward,
    bit for bit (and with the forward's per-event state sums read by both)."""
    print(f"scan_bwd_rows case B={B} D={D} L={L} p={p}/{ps} N={N} {dtype} z={with_z} expand={expand} "
          f"acc={use_acc}", flush=True)
    dev = cuda_device
    c = _expanded_case(B, D, L, p, N, dtype, L + N + expand, with_z, ps, expand)
    NC = B * D
    cud = lambda x: None if x is None else x.to(dev)
    k_t, cu_t = torch.from_numpy(c["k"]).to(dev), torch.from_numpy(c["cu"]).to(dev)
    args = (cud(c["u"]), k_t, cu_t, c["ms"], cud(c["dt_i"]), cud(c["dt_a"]), cud(c["A"]), cud(c["WB"]), cud(c["WC"]))
    acc = torch.empty(len(c["k"]), dtype=torch.float32, device=dev) if use_acc else None
    res = ssc.fwd_flat_ch(*args, D=cud(c["D"]), z=cud(c["z"]), is_depthwise_bc=True, _acc=acc)
    kw = dict(D=cud(c["D"]), z=cud(c["z"]), out=res[0] if with_z else None, is_depthwise_bc=True, _acc=acc)
    g_plain = ssc.bwd_flat_ch(*args, cud(c["dout"]), res[1], **kw)
    bitmask, tile_start = _index(c, NC, L, dev, expand)
    dx = torch.full((NC, L), float("nan"), dtype=dtype, device=dev)  # every element must be written
    g_rows = ssc.bwd_flat_ch(*args, cud(c["dout"]), res[1], **kw, _rows=(bitmask, expand, tile_start, dx))
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(g_plain, g_rows)):
        assert torch.equal(a, b), f"gradient {i} differs"
    # the gather backward of du, on the CPU
    ref = torch.zeros(NC, L, dtype=dtype)
    ch = np.repeat(np.arange(NC), np.diff(c["cu"]))
    ref[torch.from_numpy(ch).long(), torch.from_numpy(c["t"]).long()] = g_plain[0].cpu()
    assert torch.equal(dx.cpu(), ref)
