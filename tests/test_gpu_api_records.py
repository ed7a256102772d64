"""The drop-in API path reads what the extraction recorded on its outputs
(the event index on t_steps, the longest channel on cu_seqlens) instead of
recomputing it: restore forward / backward from the extraction's index (the
backward in one kernel where it fits one launch), the gather backward row by
row, the scan without its length report. Against the same path on copies of
those tensors (no records: index rebuilt, zero-fill + scatter, two-pass
restore backward, the report read), every result agrees."""
import pytest
import torch

from bc_mamba_amd import _provenance as prov
from bc_mamba_amd import e_model
from bc_mamba_amd import extract_events_cuda as ee
from bc_mamba_amd import restore_dense_cuda_nodecay as rdc
from bc_mamba_amd.selective_scan_interface import selective_scan_flat_ch_fn
from bc_mamba_amd.workloads import make_workload
from conftest import assert_close

pytestmark = pytest.mark.gpu


def _path(w, strip):
    x_conv = w.x_conv.detach().clone().requires_grad_(True)
    params = [p.detach().clone().requires_grad_(True) for p in (w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C, w.D_skip)]
    ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane, w.threshold)
    if strip:
        ch, t, cu = ch.clone(), t.clone(), cu.clone()
        assert prov.event_index_for(t, cu, w.L) is None and prov.max_seqlen_of(cu) is None
    else:
        assert prov.event_index_for(t, cu, w.L, ch) is not None and prov.max_seqlen_of(cu) == int(ms)
    u = e_model.GatherEventsFn.apply(x_conv, ch, t)
    y, _ = selective_scan_flat_ch_fn(u, k, cu, int(ms), *params[:5], D=params[5], is_depthwise_bc=True)
    out = e_model.restore_dense_fn(y, t, cu, w.D, w.L)
    out.backward(w.dout)
    return out.detach(), y.detach(), [x_conv.grad] + [p.grad for p in params]


@pytest.mark.parametrize("cfg", [0, 1])
def test_api_path_with_records_matches_without(cuda_device, cfg):
    print(f"api records: config {cfg}", flush=True)
    w = make_workload(cfg).to(cuda_device)
    out_r, y_r, g_r = _path(w, strip=False)
    out_s, y_s, g_s = _path(w, strip=True)
    torch.cuda.synchronize()
    assert torch.equal(y_r, y_s)
    assert torch.equal(out_r, out_s)  # the same index, built twice
    # dy: the one-kernel restore backward sums runs that cross two or more
    # tile edges in another order than the two-pass form (fp32 rounding)
    for name, a, b in zip(("x_conv", "dt_idle", "dt_active", "A", "W_B", "W_C", "D"), g_r, g_s):
        assert_close(a.cpu(), b.cpu().numpy(), 1e-5, 1e-6, name)


def test_extraction_index_equals_built_index(cuda_device):
    w = make_workload(1, B=4).to(cuda_device)
    ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane, w.threshold)
    bm, ts = prov.event_index_for(t, cu, w.L)
    bm2, ts2 = rdc.build_event_index(t, cu, w.L)
    assert torch.equal(bm, bm2) and torch.equal(ts, ts2)
    assert int(ms) == int((cu[1:] - cu[:-1]).max())


def test_changed_streams_fall_back(cuda_device):
    w = make_workload(0).to(cuda_device)
    ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane, w.threshold)
    y = torch.randn(t.numel(), device=cuda_device)
    before = rdc.restore_dense_fwd(y, t, cu, w.D, w.L)
    # move every channel's first event one step earlier where it can: the
    # same tensor edited in place, still sorted per channel; the extraction's
    # index no longer describes it and must not be used
    first = cu[:-1][cu[1:] > cu[:-1]].long()
    first = first[t[first] > 0]
    assert first.numel() > 0
    t[first] -= 1
    assert prov.event_index_for(t, cu, w.L) is None
    got = rdc.restore_dense_fwd(y, t, cu, w.D, w.L)
    exp = rdc.restore_dense_fwd(y, t.clone(), cu.clone(), w.D, w.L)
    assert torch.equal(got, exp) and not torch.equal(got, before)
    dout = torch.randn_like(got)
    assert torch.equal(rdc.restore_dense_bwd(dout, t, cu, w.D, w.L), rdc.restore_dense_bwd(dout, t.clone(), cu.clone(),
                                                                                           w.D, w.L))


def test_understated_max_seqlen_still_reported(cuda_device):
    w = make_workload(0).to(cuda_device)
    ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane, w.threshold)
    u = ee.gather_events_fwd(w.x_conv, ch, t)[0]
    with pytest.raises(RuntimeError, match="more than max_seqlen"):
        selective_scan_flat_ch_fn(u, k, cu, int(ms) - 1, w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C, D=w.D_skip,
                                  is_depthwise_bc=True)


def test_restore_backward_sync_area_reuse(cuda_device):
    """The one-kernel restore backward's per-stream sync area is reused and
    grown across calls of other sizes (each call leaves it zero): small,
    large, small again, each against the two-pass form on copies."""
    for cfg, B in ((0, None), (1, 8), (0, None), (1, 4)):
        w = make_workload(cfg, **({} if B is None else {"B": B})).to(cuda_device)
        ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane, w.threshold)
        assert prov.event_index_for(t, cu, w.L) is not None
        got = rdc.restore_dense_bwd(w.dout, t, cu, w.D, w.L)
        ref = rdc.restore_dense_bwd(w.dout, t.clone(), cu.clone(), w.D, w.L)
        assert_close(got.cpu(), ref.cpu().numpy(), 1e-5, 1e-6, f"dy config {cfg} B={B}")
    areas = [a for (dev, _), a in rdc._sync_areas.items() if dev == cuda_device.index]
    assert areas and all(int(a.abs().sum()) == 0 for a in areas)  # left zero


def test_api_path_without_events(cuda_device):
    """A membrane with no event: the extraction records its (zero) longest
    channel and no index; the API path runs and gives a zero output and
    zero input gradient."""
    w = make_workload(0).to(cuda_device)
    w.membrane = torch.zeros_like(w.membrane)
    ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane, w.threshold)
    assert ch.numel() == 0 and int(ms.max()) == 0 and prov.max_seqlen_of(cu) == 0
    x_conv = w.x_conv.detach().clone().requires_grad_(True)
    params = [p.detach().clone().requires_grad_(True) for p in (w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C, w.D_skip)]
    u = e_model.GatherEventsFn.apply(x_conv, ch, t)
    y, _ = selective_scan_flat_ch_fn(u, k, cu, int(ms.max()), *params[:5], D=params[5], is_depthwise_bc=True)
    out = e_model.restore_dense_fn(y, t, cu, w.D, w.L)
    out.backward(w.dout)
    torch.cuda.synchronize()
    assert out.shape == (w.B, w.L, w.D) and int(torch.count_nonzero(out)) == 0
    assert x_conv.grad is not None and int(torch.count_nonzero(x_conv.grad)) == 0


@pytest.mark.parametrize("expand", [2, 3])
def test_expanded_offsets_carry_the_maximum(cuda_device, expand):
    """expand_base_events copies the base offsets' recorded maximum to the
    logical offsets (every logical channel holds its base channel's events),
    and the scan over them needs no length report."""
    w = make_workload(0).to(cuda_device)
    B, Dm = w.B, w.D
    bch, bt, bk, bcu, _, bms = ee.extract_base_events(w.membrane, w.threshold)
    ch, t, k, cu, ms = ee.expand_base_events(bch, bt, bk, bcu, B, Dm, expand)
    assert prov.max_seqlen_of(cu) == int(ms) == int(bms)
    assert prov.event_index_for(t, cu, w.L) is None  # the expanded streams carry no index
    lens = (cu[1:] - cu[:-1]).max()
    assert int(lens) == int(ms)
