"""GPU parity of the one-kernel restore backward (bcm_restore_bwd_chained):
against the CPU oracle, against the two-pass bcm_restore_bwd on the same
event index (bit-equal for every run that crosses at most one 64-step tile
edge, where both add the same two partials), and the sync area's contract
(all zero again after every call, so one area serves call after call)."""
import numpy as np
import pytest
import torch

from bc_mamba_amd import _native as nat
from bc_mamba_amd import restore_dense_cuda_nodecay as rd
from bc_mamba_amd.workloads import _markov_events
from conftest import assert_close
from oracle import event_path as orc

pytestmark = pytest.mark.gpu


def _sync(n_ch, L, dev):
    return torch.zeros(nat.lib().bcm_restore_bwd_sync_bytes(n_ch, L) // 8, dtype=torch.int64, device=dev)


def _chained(dout, index, n_ch, dim, L, n_events, sync):
    bm, ts, mrd = index
    dy = torch.full((n_events,), float("nan"), device=dout.device)  # every entry must be written
    nat.call("bcm_restore_bwd_chained", nat.ptr(dout), nat.dtype_code(dout.dtype), nat.ptr(bm), int(mrd),
             nat.ptr(ts), n_ch, dim, L, nat.ptr(dy), nat.dtype_code(dy.dtype), n_events, nat.ptr(sync),
             8 * sync.numel(), nat.stream_of(dout))
    return dy


def _two_pass(dout, index, n_ch, dim, L, n_events):
    dy = torch.full((n_events,), float("nan"), device=dout.device)
    rd.restore_bwd_indexed(dout, index, n_ch, dim, L, dy)
    return dy


def _edges_crossed(t, cu, L):
    """Tile edges inside each event's run [t_e, t_next) (t_next: the
    channel's next event or L)."""
    t = t.astype(np.int64)
    nxt = np.empty_like(t)
    nxt[:-1] = t[1:]
    ends = cu[1:].astype(np.int64) - 1
    ends = ends[cu[1:] > cu[:-1]]
    nxt[ends] = L
    return (nxt - 1) // 64 - t // 64


def _steps(v, dev):  # the index builder takes a non-null step array even without events
    return torch.from_numpy(v if len(v) else np.zeros(1, np.int32)).to(dev)


def _check(mem, L, dim, dtype, dev, seed, sync=None, mrd=1, base=None):
    """Chained vs oracle and two-pass on the events of `mem` (n_ch, L); with
    mrd > 1 the bitmask rows are those of `base` (groups of mrd channels
    share one, the expand layout)."""
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem.numpy()[None], 0.5)
    n_ch, E = mem.shape[0], len(t)
    cu_d = torch.from_numpy(cu).to(dev)
    bm, ts = rd.build_event_index(_steps(t, dev), cu_d, L)
    if mrd > 1:
        bch, bt, _, bcu, _, _ = orc.extract_base_events(base.numpy(), 0.5)
        bm, _ = rd.build_event_index(_steps(bt, dev), torch.from_numpy(bcu).to(dev), L)
    index = (bm, ts, mrd)
    g = torch.Generator().manual_seed(seed)
    dout = torch.randn(n_ch // dim, L, dim, generator=g).to(dtype)
    dout_d = dout.to(dev)
    if sync is None:
        sync = _sync(n_ch, L, dev)
    dy = _chained(dout_d, index, n_ch, dim, L, E, sync)
    ref2 = _two_pass(dout_d, index, n_ch, dim, L, E)
    torch.cuda.synchronize()
    assert torch.count_nonzero(sync).item() == 0, "sync area not left zero"
    dyc = dy.cpu()
    assert not torch.isnan(dyc).any(), "an event's entry was not written"
    assert_close(dyc, orc.restore_bwd(dout.float().numpy(), t, cu, dim, L), 1e-5, 1e-6, "dy")
    one_edge = torch.from_numpy(_edges_crossed(t, cu, L) <= 1)
    assert torch.equal(dyc[one_edge], ref2.cpu()[one_edge]), "runs within one tile edge differ from the two-pass form"
    assert_close(dyc, ref2.cpu(), 1e-5, 1e-6, "dy vs two-pass")
    return E, int((~one_edge).sum())


CASES = [  # B, D, L, density
    (2, 256, 2048, 0.15),  # config-1 channel layout, fewer batches
    (2, 100, 500, 0.3),    # D not a multiple of 64
    (3, 7, 65, 0.5),       # ragged last tile
    (1, 3, 1, 0.9),
    (1, 2, 6000, 0.9),     # > 4095 events per channel
    (2, 64, 300, 0.02),
    (1, 64, 256, 0.6),     # > 1024 events per 64-channel tile: the direct-store path
    (2, 130, 3000, 0.004),  # long silences: most runs cross several tile edges
]


@pytest.mark.parametrize("B,D,L,p", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_restore_bwd_chained(cuda_device, B, D, L, p, dtype):
    print(f"chained restore bwd B={B} D={D} L={L} p={p} {dtype}", flush=True)
    g = torch.Generator().manual_seed(L + D)
    mem = (torch.rand(B * D, L, generator=g) < p).float()
    mem[::5] = 0.0  # empty channels
    _check(mem, L, D, dtype, cuda_device, seed=B + L)


def test_restore_bwd_chained_markov_many_rounds(cuda_device):
    """Config 3's bursty law at its tile grid (B64 D128 L4000: 8064 waves,
    more than 4 blocks per CU, so two launches): long silences, chains of
    tiles without events, walks back across the launch boundary."""
    print("chained restore bwd markov B64 D128 L4000", flush=True)
    g = torch.Generator().manual_seed(11)
    mem = _markov_events(g, 64 * 128, 4000).float()
    E, long_runs = _check(mem, 4000, 128, torch.float32, cuda_device, seed=3)
    assert long_runs > 1000  # the look-back walked past eventless tiles


def test_restore_bwd_chained_expand_layout(cuda_device):
    """mask_row_div 2: pairs of channels share one bitmask row."""
    print("chained restore bwd expand layout", flush=True)
    B, D, L, mrd = 2, 192, 1000, 2
    g = torch.Generator().manual_seed(4)
    base = (torch.rand(B, D // mrd, L, generator=g) < 0.05).float()
    base.view(-1, L)[::7] = 0.0
    mem = base.repeat_interleave(mrd, dim=1).reshape(B * D, L)
    _check(mem, L, D, torch.float32, cuda_device, seed=9, mrd=mrd, base=base)


def test_restore_bwd_chained_reuses_sync(cuda_device):
    """One sync area, three calls in a row on different shapes (the second
    smaller): each result right, the area zero after each."""
    sync = _sync(4 * 256, 2048, cuda_device)
    for i, (B, D, L, p) in enumerate([(4, 256, 2048, 0.1), (1, 70, 700, 0.01), (4, 256, 2048, 0.2)]):
        print(f"chained restore bwd reuse call {i}: B={B} D={D} L={L} p={p}", flush=True)
        g = torch.Generator().manual_seed(20 + i)
        mem = (torch.rand(B * D, L, generator=g) < p).float()
        _check(mem, L, D, torch.float32, cuda_device, seed=i, sync=sync)


def test_restore_bwd_chained_no_events(cuda_device):
    B, D, L = 2, 3, 100
    mem = torch.zeros(B * D, L)
    sync = _sync(B * D, L, cuda_device)
    bm, ts = rd.build_event_index(_steps(np.zeros(0, np.int32), cuda_device),
                                  torch.zeros(B * D + 1, dtype=torch.int32, device=cuda_device), L)
    dout = torch.randn(B, L, D, device=cuda_device)
    dy = _chained(dout, (bm, ts, 1), B * D, D, L, 0, sync)
    assert dy.numel() == 0 and torch.count_nonzero(sync).item() == 0
    assert mem.sum() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_restore_bwd_chained_16bit_dy(cuda_device, dtype):
    """dy stored in dout's 16-bit dtype: the fp32 dy of the same kernel,
    rounded as torch rounds it (bit-equal), every entry written."""
    print(f"chained restore bwd 16-bit dy {dtype}", flush=True)
    B, D, L = 2, 256, 2048
    g = torch.Generator().manual_seed(31)
    mem = (torch.rand(B * D, L, generator=g) < 0.1).float()
    mem[::7] = 0.0
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem.numpy()[None], 0.5)
    E = len(t)
    bm, ts = rd.build_event_index(_steps(t, cuda_device), torch.from_numpy(cu).to(cuda_device), L)
    dout = torch.randn(B, L, D, generator=g).to(dtype).to(cuda_device)
    sync = _sync(B * D, L, cuda_device)
    dy32 = _chained(dout, (bm, ts, 1), B * D, D, L, E, sync)
    dy16 = torch.full((E,), float("nan"), dtype=dtype, device=cuda_device)
    nat.call("bcm_restore_bwd_chained", nat.ptr(dout), nat.dtype_code(dtype), nat.ptr(bm), 1, nat.ptr(ts), B * D, D,
             L, nat.ptr(dy16), nat.dtype_code(dtype), E, nat.ptr(sync), 8 * sync.numel(), nat.stream_of(dout))
    torch.cuda.synchronize()
    assert torch.count_nonzero(sync).item() == 0
    assert not torch.isnan(dy16).any()
    assert torch.equal(dy16.cpu(), dy32.cpu().to(dtype))
