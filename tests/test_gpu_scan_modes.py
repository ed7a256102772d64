"""GPU parity of the non-depthwise B/C modes of fwd_flat_ch / bwd_flat_ch
(selective_scan.cpp:760-776, 840-848, 969-990, 1085-1090) against the CPU
oracle: legacy per-event [dstate, E] B/C, legacy per-model-channel
[dstate, dim] B/C in the backward, the tiled [n_tiles, dstate, T] layout,
and depthwise + pointwise pw_B / pw_C mixing. fp32 within rtol 1e-4, bf16
within 2e-2."""
import math

import numpy as np
import pytest
import torch

from bc_mamba_amd import selective_scan_cuda as ssc
from bc_mamba_amd import selective_scan_interface as ssi
from conftest import assert_close
from oracle import event_path as orc

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-4, 1e-6), torch.bfloat16: (2e-2, 2e-3)}


def _case(B, D, L, p, N, dtype, seed, with_z=False, with_D=True, empty_every=0):
    g = torch.Generator().manual_seed(seed)
    mem = (torch.rand(B, D, L, generator=g) < p).float()
    if empty_every:
        mem.view(B * D, L)[::empty_every] = 0.0
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem.numpy(), 0.5)
    E = len(ch)
    c = dict(ch=ch, k=k, cu=cu, ms=ms, dim=D, N=N, E=E)
    c["u"] = torch.randn(E, generator=g).to(dtype)
    c["dout"] = torch.randn(E, generator=g).to(dtype)
    c["z"] = torch.randn(E, generator=g).to(dtype) if with_z else None
    c["dt_i"] = torch.nn.functional.softplus(torch.randn(D, generator=g) - 2.0)
    c["dt_a"] = torch.nn.functional.softplus(torch.randn(D, generator=g) - 2.0)
    c["A"] = -torch.exp(torch.rand(D, N, generator=g) * math.log(16.0))
    c["D"] = torch.randn(D, generator=g) if with_D else None
    c["g"] = g
    return c


def _np(x):
    return None if x is None else x.float().cpu().numpy()


def _check_fwd_bwd(c, B, C, dtype, dev, tile_offsets=None, T=0, bwd_B=None, bwd_C=None):
    """Forward with (B, C), backward with (bwd_B or B, bwd_C or C); both against
    the oracle on the per-event values of the same operands."""
    cud = lambda x: None if x is None else x.to(dev)
    k_t, cu_t = torch.from_numpy(c["k"]).to(dev), torch.from_numpy(c["cu"]).to(dev)
    to_t = None if tile_offsets is None else torch.from_numpy(tile_offsets.astype(np.int32)).to(dev)
    common = (cud(c["u"]), k_t, cu_t, c["ms"], cud(c["dt_i"]), cud(c["dt_a"]), cud(c["A"]))
    kw = dict(tile_offsets=to_t, tile_chunk_size=T, is_depthwise_bc=False)
    rtol, atol = TOL[dtype]
    pe = lambda X: orc.bc_per_event(_np(X), c["cu"], c["dim"], c["N"], tile_offsets if to_t is not None else None, T)
    res = ssc.fwd_flat_ch(*common, cud(B), cud(C), D=cud(c["D"]), z=cud(c["z"]), **kw)
    ref = orc.scan_var_fwd(_np(c["u"]), c["k"], c["cu"], c["ms"], _np(c["dt_i"]), _np(c["dt_a"]), _np(c["A"]),
                           pe(B), pe(C), _np(c["D"]), _np(c["z"]))
    assert res[0].dtype == dtype
    assert_close(res[0].float().cpu(), ref[0], rtol, atol, "out")
    assert_close(res[1].cpu(), ref[1], rtol, atol, "x")
    if c["z"] is not None:
        assert_close(res[2].float().cpu(), ref[2], rtol, atol, "out_z")
    Bb = B if bwd_B is None else bwd_B
    Cb = C if bwd_C is None else bwd_C
    gb = ssc.bwd_flat_ch(*common, cud(Bb), cud(Cb), cud(c["dout"]), res[1], D=cud(c["D"]), z=cud(c["z"]),
                         out=res[0] if c["z"] is not None else None, **kw)
    out_used = res[0].float().cpu().numpy() if c["z"] is not None else None
    gref = orc.scan_var_bwd(_np(c["u"]), c["k"], c["cu"], c["ms"], _np(c["dt_i"]), _np(c["dt_a"]), _np(c["A"]),
                            pe(Bb), pe(Cb), _np(c["dout"]), _np(c["D"]), _np(c["z"]), out_used)
    lay = lambda G, X: orc.bc_grad_layout(G, tuple(X.shape), c["cu"], c["dim"],
                                          tile_offsets if to_t is not None else None, T)
    assert gb[2].shape == Bb.shape and gb[3].shape == Cb.shape
    for name, got, want in [("du", gb[0], gref[0]), ("dA", gb[1], gref[1]), ("dB", gb[2], lay(gref[2], Bb)),
                            ("dC", gb[3], lay(gref[3], Cb)), ("ddt_idle", gb[4], gref[4]),
                            ("ddt_active", gb[5], gref[5])]:
        assert_close(got.float().cpu(), want, rtol, atol, name)
    i = 6
    if c["D"] is not None:
        assert_close(gb[i].cpu(), gref[6], rtol, atol, "dD")
        i += 1
    if c["z"] is not None:
        assert_close(gb[i].float().cpu(), gref[7], rtol, atol, "dz")
    return res, gb


@pytest.mark.parametrize("with_z", [False, True])
@pytest.mark.parametrize("shape", [(2, 8, 300, 0.3, 4), (1, 4, 5000, 0.6, 16)])
def test_legacy_per_event_bc(cuda_device, shape, with_z):
    """[dstate, E] B/C; the second shape has channels over 2048 events (two
    saved-state chunks) and passes that end mid-chunk."""
    B_, D, L, p, N = shape
    c = _case(B_, D, L, p, N, torch.float32, 11 + N, with_z=with_z)
    Bt = torch.randn(N, c["E"], generator=c["g"])
    Ct = torch.randn(N, c["E"], generator=c["g"])
    _check_fwd_bwd(c, Bt, Ct, torch.float32, cuda_device)


def test_legacy_strided_rows_and_empty_channels(cuda_device):
    """B/C rows with a stride above E (slices of a wider tensor) and channels
    without events."""
    c = _case(2, 6, 200, 0.25, 8, torch.float32, 5, empty_every=3)
    Bw = torch.randn(8, c["E"] + 37, generator=c["g"])
    Cw = torch.randn(8, c["E"] + 5, generator=c["g"])
    Bt, Ct = Bw[:, 3:3 + c["E"]], Cw[:, :c["E"]]
    assert Bt.stride(0) != c["E"]
    _check_fwd_bwd(c, Bt, Ct, torch.float32, cuda_device)


@pytest.mark.parametrize("which", ["B", "C", "BC"])
def test_legacy_per_channel_bc_backward(cuda_device, which):
    """The backward also takes [dstate, dim] B and/or C (one value per model
    channel; selective_scan.cpp:985-989, :304-305); dB/dC are then sums over
    the events of each model channel."""
    c = _case(2, 4, 400, 0.3, 6, torch.float32, 21)
    Bt = torch.randn(6, c["E"], generator=c["g"])
    Ct = torch.randn(6, c["E"], generator=c["g"])
    Bd = torch.randn(6, 4, generator=c["g"])
    Cd = torch.randn(6, 4, generator=c["g"])
    # forward on the per-event expansion of the same values, so x matches
    pe = lambda X: torch.from_numpy(orc.bc_per_event(X.numpy(), c["cu"], 4, 6).T.copy()).float()
    fB = pe(Bd) if "B" in which else Bt
    fC = pe(Cd) if "C" in which else Ct
    _check_fwd_bwd(c, fB, fC, torch.float32, cuda_device, bwd_B=Bd if "B" in which else None,
                   bwd_C=Cd if "C" in which else None)


@pytest.mark.parametrize("T", [128, 256, 100])
def test_tiled_bc(cuda_device, T):
    """Tiled [n_tiles, dstate, T]: channel ch's events at p go to tile
    tile_offsets[ch] + p // T, column p % T (selective_scan_fwd_kernel.cuh
    :580-587); tile_offsets is the prefix sum of per-channel tile counts,
    here with one unused leading tile. dB/dC stay zero where no event maps."""
    c = _case(2, 4, 700, 0.4, 8, torch.float32, 31 + T)
    n = np.diff(c["cu"])
    tiles = (n + T - 1) // T
    toff = 1 + np.concatenate([[0], np.cumsum(tiles)])[:-1]
    nt = int(1 + tiles.sum())
    Bt = torch.randn(nt, 8, T, generator=c["g"])
    Ct = torch.randn(nt, 8, T, generator=c["g"])
    _, gb = _check_fwd_bwd(c, Bt, Ct, torch.float32, cuda_device, tile_offsets=toff, T=T)
    assert float(gb[2][0].abs().max()) == 0.0  # the unused tile


def test_legacy_bf16(cuda_device):
    c = _case(2, 8, 400, 0.3, 8, torch.bfloat16, 41, with_z=True)
    Bt = torch.randn(8, c["E"], generator=c["g"])
    Ct = torch.randn(8, c["E"], generator=c["g"])
    _check_fwd_bwd(c, Bt, Ct, torch.bfloat16, cuda_device)


@pytest.mark.parametrize("with_z", [False, True])
def test_pointwise_mixing(cuda_device, with_z):
    """Depthwise + pw_B / pw_C: W_eff = pw @ W; returns dW_B, dW_C and, last,
    dpw_B, dpw_C (selective_scan.cpp:1142-1150)."""
    dev = cuda_device
    c = _case(2, 8, 300, 0.3, 16, torch.float32, 51, with_z=with_z)
    WB = torch.randn(8, 16, generator=c["g"]) / 4.0
    WC = torch.randn(8, 16, generator=c["g"]) / 4.0
    pwB = torch.randn(8, 8, generator=c["g"]) / math.sqrt(8)
    pwC = torch.randn(8, 8, generator=c["g"]) / math.sqrt(8)
    cud = lambda x: None if x is None else x.to(dev)
    k_t, cu_t = torch.from_numpy(c["k"]).to(dev), torch.from_numpy(c["cu"]).to(dev)
    common = (cud(c["u"]), k_t, cu_t, c["ms"], cud(c["dt_i"]), cud(c["dt_a"]), cud(c["A"]), cud(WB), cud(WC))
    kw = dict(is_depthwise_bc=True, pw_B=cud(pwB), pw_C=cud(pwC))
    res = ssc.fwd_flat_ch(*common, D=cud(c["D"]), z=cud(c["z"]), **kw)
    WBe, WCe = orc.pw_effective(pwB.numpy(), WB.numpy()), orc.pw_effective(pwC.numpy(), WC.numpy())
    ref = orc.scan_fwd(_np(c["u"]), c["k"], c["cu"], c["ms"], _np(c["dt_i"]), _np(c["dt_a"]), _np(c["A"]), WBe, WCe,
                       _np(c["D"]), _np(c["z"]))
    rtol, atol = TOL[torch.float32]
    assert_close(res[0].cpu(), ref[0], rtol, atol, "out")
    assert_close(res[1].cpu(), ref[1], rtol, atol, "x")
    gb = ssc.bwd_flat_ch(*common, cud(c["dout"]), res[1], D=cud(c["D"]), z=cud(c["z"]),
                         out=res[0] if with_z else None, **kw)
    out_used = res[0].cpu().numpy() if with_z else None
    gref = orc.scan_bwd(_np(c["u"]), c["k"], c["cu"], c["ms"], _np(c["dt_i"]), _np(c["dt_a"]), _np(c["A"]), WBe,
                        WCe, _np(c["dout"]), _np(c["D"]), _np(c["z"]), out_used)
    dWB, dpwB = orc.pw_grads(pwB.numpy(), WB.numpy(), gref[2])
    dWC, dpwC = orc.pw_grads(pwC.numpy(), WC.numpy(), gref[3])
    assert len(gb) == 6 + 1 + int(with_z) + 2
    for name, got, want in [("du", gb[0], gref[0]), ("dA", gb[1], gref[1]), ("dW_B", gb[2], dWB),
                            ("dW_C", gb[3], dWC), ("ddt_idle", gb[4], gref[4]), ("ddt_active", gb[5], gref[5]),
                            ("dD", gb[6], gref[6]), ("dpw_B", gb[-2], dpwB), ("dpw_C", gb[-1], dpwC)]:
        assert_close(got.cpu(), want, rtol, atol, name)


def test_autograd_legacy_mode(cuda_device):
    """selective_scan_flat_ch_fn routes the legacy mode's dB / dC into the
    B / C inputs' .grad."""
    dev = cuda_device
    c = _case(2, 4, 300, 0.3, 8, torch.float32, 61)
    Bt = torch.randn(8, c["E"], generator=c["g"]).to(dev).requires_grad_(True)
    Ct = torch.randn(8, c["E"], generator=c["g"]).to(dev).requires_grad_(True)
    u = c["u"].to(dev).requires_grad_(True)
    A = c["A"].to(dev).requires_grad_(True)
    y, x = ssi.selective_scan_flat_ch_fn(u, torch.from_numpy(c["k"]).to(dev), torch.from_numpy(c["cu"]).to(dev),
                                         c["ms"], c["dt_i"].to(dev), c["dt_a"].to(dev), A, Bt, Ct,
                                         D=c["D"].to(dev), is_depthwise_bc=False)
    y.backward(c["dout"].to(dev))
    pe = lambda X: X.detach().cpu().numpy().T
    gref = orc.scan_var_bwd(_np(c["u"]), c["k"], c["cu"], c["ms"], _np(c["dt_i"]), _np(c["dt_a"]), _np(c["A"]),
                            pe(Bt), pe(Ct), _np(c["dout"]), _np(c["D"]))
    rtol, atol = TOL[torch.float32]
    assert_close(u.grad.cpu(), gref[0], rtol, atol, "du")
    assert_close(A.grad.cpu(), gref[1], rtol, atol, "dA")
    assert_close(Bt.grad.cpu(), gref[2].T, rtol, atol, "dB")
    assert_close(Ct.grad.cpu(), gref[3].T, rtol, atol, "dC")
