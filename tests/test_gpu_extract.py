"""GPU parity of stage 1 (extraction, expansion, gather fwd/bwd) against the
CPU oracle: every index output bit-exact."""
import numpy as np
import pytest
import torch

from bc_mamba_amd import extract_events_cuda as ee
from oracle import event_path as orc

pytestmark = pytest.mark.gpu

I32 = torch.int32


def _membrane(B, Dm, L, p, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if p == "gauss":
        m = torch.randn(B, Dm, L, generator=g)
    else:
        m = (torch.rand(B, Dm, L, generator=g) < p).float()
    return m.to(dtype)


def _np(t):
    return t.detach().cpu().numpy()


CASES = [  # B, Dm, L, density, dtype
    (2, 64, 1024, "gauss", torch.float32),    # config 0 shape
    (2, 8, 2048, 0.15, torch.float32),
    (3, 5, 1, 0.5, torch.float32),
    (2, 3, 31, 0.5, torch.float32),
    (2, 3, 33, 0.5, torch.float32),
    (1, 7, 257, 0.3, torch.float32),
    (2, 4, 1000, 0.05, torch.float32),
    (1, 3, 4097, 0.6, torch.float32),
    (2, 6, 777, "gauss", torch.bfloat16),
    (2, 6, 1024, "gauss", torch.float16),
    (1, 4, 3000, 1.0, torch.float32),
]


@pytest.mark.parametrize("B,Dm,L,p,dtype", CASES)
def test_extract_base_events_bit_exact(cuda_device, B, Dm, L, p, dtype):
    mem = _membrane(B, Dm, L, p, dtype, seed=B * 1000 + L)
    print(f"extract case B={B} Dm={Dm} L={L} p={p} {dtype}", flush=True)
    ch, t, k, cu, counts, ms = ee.extract_base_events(mem.to(cuda_device), 0.5)
    och, ot, ok, ocu, ocounts, oms = orc.extract_base_events(mem.float().numpy(), 0.5)
    assert ch.dtype == t.dtype == k.dtype == cu.dtype == I32
    for name, a, b in (("ch", ch, och), ("t", t, ot), ("k", k, ok), ("cu", cu, ocu), ("counts", counts, ocounts)):
        assert np.array_equal(_np(a), b), name
    assert ms.dim() == 0 and int(ms) == oms


def test_extract_no_events(cuda_device):
    mem = torch.zeros(2, 3, 50, device=cuda_device)
    ch, t, k, cu, counts, ms = ee.extract_base_events(mem, 0.5)
    assert ch.numel() == t.numel() == k.numel() == 0
    assert _np(cu).tolist() == [0] * 7 and _np(counts).tolist() == [0] * 6
    assert tuple(ms.shape) == (1,) and int(ms[0]) == 0  # the reference returns zeros({1}) here


def test_extract_threshold_is_strict_fp32(cuda_device):
    x = torch.tensor([[[0.5, 0.50000006, 0.49999997, 2.0, 0.5]]], device=cuda_device)
    ch, t, k, cu, counts, ms = ee.extract_base_events(x, 0.5)
    assert _np(t).tolist() == [1, 3] and _np(k).tolist() == [2, 2]


@pytest.mark.parametrize("expand", [1, 2, 3])
def test_expand_base_events(cuda_device, expand):
    B, Dm, L = 2, 5, 300
    mem = _membrane(B, Dm, L, 0.2, torch.float32, 7)
    bch, bt, bk, bcu, _, _ = ee.extract_base_events(mem.to(cuda_device), 0.5)
    ch, t, k, cu, ms = ee.expand_base_events(bch, bt, bk, bcu, B, Dm, expand)
    o = orc.expand_base_events(_np(bch), _np(bt), _np(bk), _np(bcu), B, Dm, expand)
    for name, a, b in zip(("ch", "t", "k", "cu"), (ch, t, k, cu), o[:4]):
        assert np.array_equal(_np(a), b), name
    assert int(ms) == o[4]


def test_expand_empty(cuda_device):
    e = torch.zeros(0, dtype=I32, device=cuda_device)
    ch, t, k, cu, ms = ee.expand_base_events(e, e, e, torch.zeros(7, dtype=I32, device=cuda_device), 2, 3, 2)
    assert ch.numel() == 0 and _np(cu).tolist() == [0] * 13 and tuple(ms.shape) == (1,)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_gather_fwd_bwd(cuda_device, dtype):
    B, D, L = 2, 6, 513
    mem = _membrane(B, D, L, 0.2, torch.float32, 3)
    x = torch.randn(B, D, L, generator=torch.Generator().manual_seed(4)).to(dtype)
    ch, t, k, cu, _, _ = ee.extract_base_events(mem.to(cuda_device), 0.5)
    u = ee.gather_events_fwd(x.to(cuda_device), ch, t)[0]
    assert u.dtype == dtype
    ref = orc.gather_fwd(x.float().numpy(), _np(ch), _np(t))
    assert np.array_equal(_np(u.float()), ref)
    g = torch.randn(u.numel(), generator=torch.Generator().manual_seed(5)).to(dtype)
    dx = ee.gather_events_bwd(g.to(cuda_device), ch, t, B * D, L)[0]
    assert tuple(dx.shape) == (B * D, L) and dx.dtype == dtype
    assert np.array_equal(_np(dx.float()), orc.gather_bwd(g.float().numpy(), _np(ch), _np(t), B * D, L))


def test_legacy_extract_events(cuda_device):
    mask = torch.rand(2, 4, 130, generator=torch.Generator().manual_seed(9)) < 0.3
    ch, t, k, cu, ms, hf = ee.extract_events(mask.to(cuda_device))
    och, ot, ok, ocu, _, oms = orc.extract_base_events(mask.float().numpy(), 0.5)
    for a, b in ((ch, och), (t, ot), (k, ok), (cu, ocu)):
        assert np.array_equal(_np(a), b)
    first = np.ones(len(och), bool)
    first[1:] = och[1:] != och[:-1]
    assert np.array_equal(_np(hf), first.astype(np.int32)) and int(ms) == oms


def _tile_starts(t, cu, L):
    NC = len(cu) - 1
    nT = (L + 63) // 64
    out = np.zeros((NC, nT + 1), np.int64)
    for c in range(NC):
        ts = t[cu[c]:cu[c + 1]]
        out[c, :nT] = cu[c] + np.searchsorted(ts, np.arange(nT) * 64, side="left")
        out[c, nT] = cu[c + 1]
    return out


@pytest.mark.parametrize("expand,dtype,L", [(1, torch.float32, 2048), (2, torch.float32, 1000),
                                             (2, torch.bfloat16, 333), (3, torch.float16, 64)])
def test_fused_extract_matches_composition(cuda_device, expand, dtype, L):
    B, Dm = 2, 5
    mem = _membrane(B, Dm, L, 0.2, torch.float32, 11).to(cuda_device)
    x = torch.randn(B, Dm * expand, L, generator=torch.Generator().manual_seed(12)).to(dtype).to(cuda_device)
    ch, t, k, cu, ms, xe, (bitmask, tile_start, ex) = ee.extract_events_indexed(mem, 0.5, expand, x)
    bch, bt, bk, bcu, _, _ = ee.extract_base_events(mem, 0.5)
    rch, rt, rk, rcu, rms = ee.expand_base_events(bch, bt, bk, bcu, B, Dm, expand)
    for a, b in ((ch, rch), (t, rt), (k, rk), (cu, rcu)):
        assert torch.equal(a, b)
    assert ms == int(rms) and ex == expand
    assert torch.equal(xe, ee.gather_events_fwd(x, rch, rt)[0])
    assert np.array_equal(_np(tile_start), _tile_starts(_np(rt), _np(rcu), L))
    # without positions: same k, offsets, gathered values and tile table
    ch2, t2, k2, cu2, ms2, xe2, (bitmask2, tile_start2, _) = ee.extract_events_indexed(mem, 0.5, expand, x,
                                                                                      positions=False)
    assert ch2 is None and t2 is None and ms2 == ms
    assert torch.equal(k2, k) and torch.equal(cu2, cu) and torch.equal(xe2, xe)
    nw = 2 * ((L + 63) // 64)  # the words the tile masks read (the rest is row padding)
    assert torch.equal(bitmask2[:, :nw], bitmask[:, :nw]) and torch.equal(tile_start2, tile_start)


def test_gather_bwd_rows_matches_scatter(cuda_device):
    from bc_mamba_amd import _native as nat
    B, Dm, L, expand = 2, 3, 700, 2
    mem = _membrane(B, Dm, L, 0.25, torch.float32, 13).to(cuda_device)
    x = torch.randn(B, Dm * expand, L, device=cuda_device)
    ch, t, k, cu, ms, xe, (bitmask, tile_start, ex) = ee.extract_events_indexed(mem, 0.5, expand, x)
    g = torch.randn(ch.numel(), device=cuda_device)
    dx = torch.empty(B * Dm * expand, L, device=cuda_device)
    nat.call("bcm_gather_bwd_rows", nat.ptr(g), nat.F32, nat.ptr(bitmask), expand, nat.ptr(tile_start),
             B * Dm * expand, L, nat.ptr(dx), nat.stream_of(g))
    assert torch.equal(dx, ee.gather_events_bwd(g, ch, t, B * Dm * expand, L)[0])


@pytest.mark.parametrize("NC,L,p,expand", [(1, 1, 0.5, 1), (3, 100, 0.3, 1), (64, 2048, 0.15, 1), (65, 64, 0.9, 2),
                                           (1001, 333, 0.2, 1), (8192, 64, 0.15, 1), (10, 700, 0.25, 3)])
def test_block_offsets_match_scan(cuda_device, NC, L, p, expand):
    """count with per-block sums + fill deriving its own row offsets give the
    cu_seqlens, k, gathered x, tile table and (E, max) of the composition
    with the separate offsets scan."""
    from bc_mamba_amd import _native as nat
    mem = _membrane(1, NC, L, p, torch.float32, 31).to(cuda_device)
    x = torch.randn(1, NC * expand, L, generator=torch.Generator().manual_seed(32)).to(cuda_device)
    ch, t, k, cu, ms, xe, (bitmask, tile_start, _) = ee.extract_events_indexed(mem, 0.5, expand, x,
                                                                                exact_alloc=True)
    E = k.numel()
    s = nat.stream_of(mem)
    i32 = dict(dtype=torch.int32, device=cuda_device)
    bm = torch.empty((NC, nat.bitmask_words(L)), **i32)
    counts = torch.empty(NC, **i32)
    bsums = torch.empty(nat.lib().bcm_extract_block_sums_bytes(NC) // 4, **i32)
    cap = NC * expand * L
    cu2, k2 = torch.empty(NC * expand + 1, **i32), torch.empty(cap, **i32)
    xe2 = torch.empty(cap, dtype=x.dtype, device=cuda_device)
    ts2 = torch.empty_like(tile_start)
    meta = nat.HostMeta()
    meta.arm()
    nat.call("bcm_extract_count_blocks", nat.ptr(mem), nat.F32, NC, L, 0.5, nat.ptr(bm), nat.ptr(counts),
             nat.ptr(bsums), s)
    nat.call("bcm_extract_fill_blocks", nat.ptr(bm), nat.ptr(counts), nat.ptr(bsums), meta.ptr(), NC, L, expand,
             nat.ptr(x), nat.F32, nat.ptr(cu2), None, None, nat.ptr(k2), nat.ptr(xe2), nat.ptr(ts2), s)
    E2, ms2 = meta.wait(torch.cuda.current_stream(cuda_device))
    assert E2 * expand == E and ms2 == ms
    assert torch.equal(cu2, cu) and torch.equal(k2[:E], k) and torch.equal(xe2[:E], xe)
    assert torch.equal(ts2, tile_start)


def _tile_table(ch, t, NC, L):
    """Oracle tile table: each channel's first event index at or after step
    64j (the channel's end for j = ntiles)."""
    nT = (L + 63) // 64
    key = ch.astype(np.int64) * L + t
    j = np.minimum(np.arange(nT + 1) * 64, L)
    q = np.arange(NC, dtype=np.int64)[:, None] * L + j[None, :]
    return np.searchsorted(key, q.ravel(), side="left").reshape(NC, nT + 1).astype(np.int32)


FUSED_CASES = [  # B, Dm, L, density, expand, positions
    (32, 256, 2048, 0.15, 1, False),  # config 1: the bench's form (2048 blocks, self-derived offsets)
    (32, 256, 2048, 0.15, 1, True),
    (2, 64, 1024, "gauss", 2, False),  # the model block's expand 2
    (3, 5, 1000, 0.3, 3, True),
    (16, 1024, 128, 0.2, 1, True),     # 16384 rows: 4096 blocks, the last self-derived size
    (64, 1024, 64, 0.25, 1, False),    # 65536 rows: 16384 blocks, offsets from the block-sum scan
    (64, 1025, 96, 0.1, 2, True),      # a partial last block, L % 64 != 0, with the block-sum scan
]


@pytest.mark.parametrize("B,Dm,L,p,expand,positions", FUSED_CASES)
def test_extract_indexed_fused_matches_oracle(cuda_device, B, Dm, L, p, expand, positions):
    """The production extraction (bcm_extract_count_blocks +
    bcm_extract_fill_blocks, one host read of E, the fill deriving row
    offsets from block sums, x gathered at the events, the tile table)
    against the oracle's extract_base_events + expand_base_events +
    gather_fwd: every index output bit-exact."""
    print(f"fused extract case B={B} Dm={Dm} L={L} p={p} expand={expand} positions={positions}", flush=True)
    mem = _membrane(B, Dm, L, p, torch.float32, seed=B + Dm + L)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, Dm * expand, L, generator=g)
    ch, t, k, cu, ms, xe, (bitmask, tile_start, mrd) = ee.extract_events_indexed(
        mem.to(cuda_device), 0.5, expand, x.to(cuda_device), positions=positions)
    bch, bt, bk, bcu, _, bms = orc.extract_base_events(mem.numpy(), 0.5)
    och, ot, ok, ocu, oms = orc.expand_base_events(bch, bt, bk, bcu, B, Dm, expand)
    assert ms == oms == bms and mrd == expand
    assert k.numel() == len(ok) and k.untyped_storage().nbytes() == 4 * len(ok)  # exact size, not worst-case views
    assert np.array_equal(_np(k), ok), "k"
    assert np.array_equal(_np(cu), ocu), "cu_seqlens"
    if positions:
        assert np.array_equal(_np(ch), och) and np.array_equal(_np(t), ot), "ch / t"
    else:
        assert ch is None and t is None
    assert np.array_equal(_np(tile_start), _tile_table(och, ot, B * Dm * expand, L)), "tile table"
    assert torch.equal(xe.cpu(), x.reshape(-1, L)[torch.from_numpy(och).long(), torch.from_numpy(ot).long()])
    # the bitmask rows are those of the base membrane (bit t of row c)
    nw = (L + 31) // 32  # words past the last step are padding
    bits = _np(bitmask).view(np.uint32)[:, :nw]
    want = np.zeros_like(bits)
    np.bitwise_or.at(want, (bch, bt // 32), (np.uint32(1) << (bt % 32).astype(np.uint32)))
    assert np.array_equal(bits, want), "bitmask"
