"""GPU parity of stage 2 (flat per-channel selective scan, depthwise mode)
against the CPU oracle: forward out / out_z / saved state x and every
gradient, within rtol 1e-4 for fp32 inputs and 2e-2 for bf16/fp16 inputs."""
import math

import numpy as np
import pytest
import torch

from bc_mamba_amd import selective_scan_cuda as ssc
from bc_mamba_amd import selective_scan_interface as ssi
from conftest import assert_close
from oracle import event_path as orc

# every case under both kernel families (dstate 16, 32 and 64: the lane groups
# and the state lanes; other dstates: the lane groups twice)
pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("scan_kernel")]

TOL = {torch.float32: (1e-4, 1e-6), torch.bfloat16: (2e-2, 2e-3), torch.float16: (2e-2, 2e-3)}


def _case(B, D, L, p, N, dtype, seed, with_z=False, with_D=True, empty_every=0, dim=None, p_short=None,
          long_every=2):
    g = torch.Generator().manual_seed(seed)
    mem = (torch.rand(B, D, L, generator=g) < p).float()
    if p_short is not None:  # bursty mix: one channel in long_every keeps density p
        rows = mem.view(B * D, L)
        short = torch.arange(B * D) % long_every != 0
        rows[short] = (torch.rand(int(short.sum()), L, generator=g) < p_short).float()
    if empty_every:
        mem.view(B * D, L)[::empty_every] = 0.0
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem.numpy(), 0.5)
    dim = D if dim is None else dim
    E = len(ch)
    u = torch.randn(E, generator=g).to(dtype)
    dout = torch.randn(E, generator=g).to(dtype)
    z = torch.randn(E, generator=g).to(dtype) if with_z else None
    dt_i = torch.nn.functional.softplus(torch.randn(dim, generator=g) - 2.0)
    dt_a = torch.nn.functional.softplus(torch.randn(dim, generator=g) - 2.0)
    A = -torch.exp(torch.rand(dim, N, generator=g) * math.log(16.0))
    WB = torch.randn(dim, N, generator=g) / math.sqrt(N)
    WC = torch.randn(dim, N, generator=g) / math.sqrt(N)
    Dv = torch.randn(dim, generator=g) if with_D else None
    return dict(ch=ch, t=t, k=k, cu=cu, ms=ms, u=u, dout=dout, z=z, dt_i=dt_i, dt_a=dt_a, A=A, WB=WB, WC=WC, D=Dv)


def _run_and_check(c, dtype, dev, use_acc=False):
    """Forward and backward through the raw API against the oracle; use_acc:
    the forward keeps its per-event state sums and the backward reads them."""
    f32 = lambda x: None if x is None else x.float().numpy()
    cud = lambda x: None if x is None else x.to(dev)
    k_t = torch.from_numpy(c["k"]).to(dev)
    cu_t = torch.from_numpy(c["cu"]).to(dev)
    args = (cud(c["u"]), k_t, cu_t, c["ms"], cud(c["dt_i"]), cud(c["dt_a"]), cud(c["A"]), cud(c["WB"]), cud(c["WC"]))
    acc = torch.empty(len(c["k"]), dtype=torch.float32, device=dev) if use_acc else None
    res = ssc.fwd_flat_ch(*args, D=cud(c["D"]), z=cud(c["z"]), is_depthwise_bc=True, _acc=acc)
    ref = orc.scan_fwd(f32(c["u"]), c["k"], c["cu"], c["ms"], f32(c["dt_i"]), f32(c["dt_a"]), f32(c["A"]),
                       f32(c["WB"]), f32(c["WC"]), f32(c["D"]), f32(c["z"]))
    rtol, atol = TOL[dtype]
    assert res[0].dtype == dtype and res[1].dtype == torch.float32
    assert_close(res[0].float().cpu(), ref[0], rtol, atol, "out")
    assert_close(res[1].cpu(), ref[1], rtol, atol, "x")
    if c["z"] is not None:
        assert_close(res[2].float().cpu(), ref[2], rtol, atol, "out_z")
    gb = ssc.bwd_flat_ch(*args, cud(c["dout"]), res[1], D=cud(c["D"]), z=cud(c["z"]),
                         out=res[0] if c["z"] is not None else None, is_depthwise_bc=True, _acc=acc)
    # the backward's z-gate reads the stored (rounded) forward output
    out_used = res[0].float().cpu().numpy() if c["z"] is not None else None
    gref = orc.scan_bwd(f32(c["u"]), c["k"], c["cu"], c["ms"], f32(c["dt_i"]), f32(c["dt_a"]), f32(c["A"]),
                        f32(c["WB"]), f32(c["WC"]), f32(c["dout"]), f32(c["D"]), f32(c["z"]), out_used)
    names = ["du", "dA", "dW_B", "dW_C", "ddt_idle", "ddt_active"]
    for i, n in enumerate(names):
        assert_close(gb[i].float().cpu(), gref[i], rtol, atol, n)
    i = 6
    if c["D"] is not None:
        assert_close(gb[i].cpu(), gref[6], rtol, atol, "dD")
        i += 1
    if c["z"] is not None:
        assert_close(gb[i].float().cpu(), gref[7], rtol, atol, "dz")
    return res, gb


SHAPES = [  # B, D, L, density, N  (max_seqlen lands in each kernel-shape bucket)
    (2, 8, 100, 0.5, 16),     # <= 64
    (2, 8, 230, 0.5, 16),     # <= 128
    (2, 8, 450, 0.5, 16),     # <= 256
    (2, 8, 2048, 0.15, 16),   # <= 384 (config-1 density)
    (2, 4, 900, 0.5, 16),     # <= 512
    (1, 4, 1900, 0.5, 16),    # <= 1024
    (1, 3, 3000, 0.6, 16),    # <= 2048
    (1, 2, 6000, 0.7, 8),     # > 2048: three 2048-event chunks
    (2, 4, 300, 0.5, 1),
    (2, 4, 300, 0.5, 7),
    (2, 4, 700, 0.4, 64),
    (1, 4, 700, 0.4, 65),
    (1, 2, 300, 0.5, 256),
    # dstate 64 with 8 channels per d and channels of 1024..2048 events: the
    # widest lane groups, whose LDS use sits at the per-workgroup limit
    (8, 2, 2600, 0.6, 64),
    (8, 2, 5000, 0.7, 64),    # and two 2048-event chunks (config-3 scale)
    # no decay table and ~3000-event channels: 2048-event passes that re-seed
    # from the saved x (no chunk_g), as the reference does
    (1, 2, 6000, 0.5, 80),
    # two states per lane (dstate 32): single and multi-pass, two x chunks
    (2, 4, 700, 0.4, 32),
    (4, 2, 3000, 0.8, 32),
]


@pytest.mark.parametrize("B,D,L,p,N", SHAPES)
def test_scan_fp32(cuda_device, B, D, L, p, N):
    print(f"scan case B={B} D={D} L={L} p={p} N={N}", flush=True)
    _run_and_check(_case(B, D, L, p, N, torch.float32, seed=L + N), torch.float32, cuda_device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_z", [False, True])
def test_scan_half_inputs(cuda_device, dtype, with_z):
    _run_and_check(_case(2, 8, 1200, 0.2, 16, dtype, seed=3, with_z=with_z), dtype, cuda_device)


@pytest.mark.parametrize("with_D", [False, True])
def test_scan_z_gate_fp32(cuda_device, with_D):
    _run_and_check(_case(2, 6, 600, 0.3, 16, torch.float32, seed=5, with_z=True, with_D=with_D),
                   torch.float32, cuda_device)


def test_scan_empty_channels(cuda_device):
    _run_and_check(_case(2, 8, 500, 0.3, 16, torch.float32, seed=6, empty_every=3), torch.float32, cuda_device)


def test_scan_no_events(cuda_device):
    c = _case(1, 4, 50, 0.0, 16, torch.float32, seed=7)
    assert len(c["ch"]) == 0
    res, gb = _run_and_check(c, torch.float32, cuda_device)
    assert torch.count_nonzero(res[1]) == 0 and all(torch.count_nonzero(g) == 0 for g in gb[1:])


def test_scan_channels_not_multiple_of_dim(cuda_device):
    c = _case(1, 10, 300, 0.3, 16, torch.float32, seed=8, dim=4)  # 10 channels, d = ch % 4
    _run_and_check(c, torch.float32, cuda_device)


def test_scan_clamped_decays(cuda_device):
    c = _case(2, 4, 1500, 0.05, 16, torch.float32, seed=9)
    c["A"] = c["A"] * 600.0  # long gaps: Δ·A·log2e far below -126
    _run_and_check(c, torch.float32, cuda_device)


@pytest.mark.parametrize("use_acc", [False, True])
def test_scan_zero_and_tiny_weights(cuda_device, use_acc):
    """Model channels whose W_B W_C has a zero or tiny entry (or a W_C too
    small to invert, or a huge one): the one-state-per-lane forward runs
    its recurrence on W_B W_C g only where every entry of the model channel
    and every 1 / W_C lie within [1e-20, 1e20], and on g elsewhere; both
    against the oracle, with long channels (two 2048-event chunks of x,
    many passes of chunk_g)."""
    c = _case(2, 8, 3000, 0.8, 16, torch.float32, seed=11)
    c["WC"][0, 3] = 0.0      # one zero: that model channel falls back
    c["WB"][1, 5] = 0.0
    c["WC"][2, :] = 1e-30    # W_B W_C ~ 1e-31: falls back
    c["WC"][3, 7] = 2e-21    # 1 / W_C beyond the bound: falls back
    c["WB"][5, 2] = 1e21     # W_B W_C beyond the bound: falls back
    c["WB"][4, :] *= 1e-3    # small but far from the bounds: scaled
    _run_and_check(c, torch.float32, cuda_device, use_acc=use_acc)


@pytest.mark.parametrize("N", [16, 32, 64])
@pytest.mark.parametrize("with_z", [False, True])
@pytest.mark.parametrize("use_acc", [False, True])
def test_scan_states_per_lane(cuda_device, N, with_z, use_acc):
    """One, two and four states per lane of the state-lane kernels (dstate
    16, 32, 64; the lane groups under the other family): z gate, clamped
    long-gap decays past the table (sparse channels) and gaps within it;
    the backward rebuilding the per-event state sums or reading the
    forward's (use_acc: written by either family's forward)."""
    c = _case(2, 8, 1500, 0.15, N, torch.float32, seed=40 + N, with_z=with_z, p_short=0.01, long_every=3)
    _run_and_check(c, torch.float32, cuda_device, use_acc=use_acc)


@pytest.mark.parametrize("N", [16, 32, 64])
@pytest.mark.parametrize("kind", ["A_positive", "dt_negative"])
def test_scan_exact_products(cuda_device, kind, N):
    """Decay exponents that can be positive (A > 0 for some states, or a
    negative Δ): the saved x then carries the multiplied-out decay products
    instead of exp2 of a Δ sum (the kernels' exact path)."""
    c = _case(2, 4, 300, 0.3, N, torch.float32, seed=31)
    g = torch.Generator().manual_seed(32)
    if kind == "A_positive":  # small growth rates on a third of the states
        grow = torch.rand(c["A"].shape, generator=g) < 0.33
        c["A"] = torch.where(grow, 0.05 * torch.rand(c["A"].shape, generator=g), c["A"])
    else:  # Δ = dt_idle·(k-1) + dt_active below 0 for long gaps on two channels
        c["dt_i"] = c["dt_i"].clone()
        c["dt_i"][:2] = -0.01
    _run_and_check(c, torch.float32, cuda_device)


def test_autograd_function_matches_raw(cuda_device):
    c = _case(2, 8, 800, 0.2, 16, torch.float32, seed=10, with_z=True)
    dev = cuda_device
    leaves = {n: c[n].to(dev).requires_grad_(True) for n in ("u", "dt_i", "dt_a", "A", "WB", "WC", "D", "z")}
    k_t, cu_t = torch.from_numpy(c["k"]).to(dev), torch.from_numpy(c["cu"]).to(dev)
    out, x = ssi.selective_scan_flat_ch_fn(leaves["u"], k_t, cu_t, c["ms"], leaves["dt_i"], leaves["dt_a"],
                                           leaves["A"], leaves["WB"], leaves["WC"], D=leaves["D"], z=leaves["z"],
                                           is_depthwise_bc=True)
    assert not x.requires_grad
    out.backward(c["dout"].to(dev))
    # the autograd function keeps the forward's state sums for its backward:
    # the raw calls do the same
    acc = torch.empty(len(c["k"]), dtype=torch.float32, device=dev)
    raw = ssc.fwd_flat_ch(*(leaves[n].detach() for n in ("u",)), k_t, cu_t, c["ms"],
                          *(leaves[n].detach() for n in ("dt_i", "dt_a", "A", "WB", "WC")),
                          D=leaves["D"].detach(), z=leaves["z"].detach(), is_depthwise_bc=True, _acc=acc)
    assert torch.equal(out.detach(), raw[2])
    gb = ssc.bwd_flat_ch(leaves["u"].detach(), k_t, cu_t, c["ms"],
                         *(leaves[n].detach() for n in ("dt_i", "dt_a", "A", "WB", "WC")),
                         c["dout"].to(dev), raw[1], D=leaves["D"].detach(), z=leaves["z"].detach(), out=raw[0],
                         is_depthwise_bc=True, _acc=acc)
    for name, g in zip(("u", "A", "WB", "WC", "dt_i", "dt_a", "D", "z"), (gb[0], gb[1], gb[2], gb[3], gb[4], gb[5],
                                                                         gb[6], gb[7])):
        assert torch.equal(leaves[name].grad, g), name


def test_scan_is_deterministic(cuda_device):
    c = _case(4, 8, 1000, 0.2, 16, torch.float32, seed=11)
    r1, g1 = _run_and_check(c, torch.float32, cuda_device)
    r2, g2 = _run_and_check(c, torch.float32, cuda_device)
    assert all(torch.equal(a, b) for a, b in zip(r1, r2)) and all(torch.equal(a, b) for a, b in zip(g1, g2))


# Long channels among short ones: max_seqlen > 512 with a mean channel length
# of at most 512 selects passes shorter than the 2048-event saved-state chunk
# (16 lanes x 16 items with the decay table, 64 x 8 without), carried through
# chunk_g; x still holds the state after every 2048 events.
BURSTY = [  # B, D, L, p_long, p_short, long_every, N
    (2, 8, 1200, 0.6, 0.02, 2, 16),   # ~720-event channels: three 256-event passes
    (2, 6, 4500, 0.6, 0.01, 6, 16),   # ~2700-event channels: x has two chunks
    (2, 4, 1500, 0.5, 0.02, 2, 80),   # no decay table: 512-event passes
]


@pytest.mark.parametrize("B,D,L,p,ps,le,N", BURSTY)
def test_scan_multipass_chunk_states(cuda_device, B, D, L, p, ps, le, N):
    print(f"multipass case B={B} D={D} L={L} p={p}/{ps} every {le} N={N}", flush=True)
    c = _case(B, D, L, p, N, torch.float32, seed=L + N, p_short=ps, long_every=le, with_z=True)
    ms, E, NC = int(c["ms"]), len(c["ch"]), B * D
    assert ms > 512 and E / NC <= 512
    a = ssc._nat.ScanArgs()
    a.n_events, a.n_channels, a.dim, a.dstate, a.max_seqlen = E, NC, D, N, ms
    pass_len, n_pass, needs = ssc._nat.scan_chunking(a)
    assert needs and pass_len < 2048 and n_pass > 1
    # direct API: the backward recomputes the pass states
    _run_and_check(c, torch.float32, cuda_device)
    # ... and reading the forward's state sums, as the autograd function does
    _, gb_direct = _run_and_check(c, torch.float32, cuda_device, use_acc=True)
    # autograd: the forward's pass states (and state sums) are kept for the backward
    dev = cuda_device
    leaves = {n: c[n].to(dev).requires_grad_(True) for n in ("u", "dt_i", "dt_a", "A", "WB", "WC", "D", "z")}
    k_t, cu_t = torch.from_numpy(c["k"]).to(dev), torch.from_numpy(c["cu"]).to(dev)
    out, x = ssi.selective_scan_flat_ch_fn(leaves["u"], k_t, cu_t, ms, leaves["dt_i"], leaves["dt_a"], leaves["A"],
                                           leaves["WB"], leaves["WC"], D=leaves["D"], z=leaves["z"],
                                           is_depthwise_bc=True)
    out.backward(c["dout"].to(dev))
    for name, g in zip(("u", "A", "WB", "WC", "dt_i", "dt_a", "D", "z"), gb_direct):
        assert torch.equal(leaves[name].grad, g), name  # same pass states either way


@pytest.mark.parametrize("B,D,L,p,ps,N", [
    (96, 2, 300, 0.5, None, 16),    # 96 channels per model channel: three rounds of 32
    (64, 2, 1200, 0.6, 0.02, 16),   # bursty multi-pass, two rounds (state lanes: length-ranked)
    (64, 2, 1200, 0.6, 0.02, 64),   # the same with four states per lane (config-3 form)
    (40, 3, 900, 0.5, 0.02, 32),    # two states per lane, ranked, rounds not filled
])
def test_scan_split_workgroups(cuda_device, B, D, L, p, ps, N):
    """Few model channels with many channels each: the backward splits every
    model channel over several workgroups (bcm_scan_bwd_workspace_bytes > 0)
    and sums their parameter-gradient partials in a fixed order."""
    print(f"split case B={B} D={D} L={L} p={p}/{ps} N={N}", flush=True)
    c = _case(B, D, L, p, N, torch.float32, seed=B + L, p_short=ps)
    a = ssc._nat.ScanArgs()
    a.n_events, a.n_channels, a.dim, a.dstate, a.max_seqlen = len(c["ch"]), B * D, D, N, int(c["ms"])
    a.n_chunks, a.dtype = max(1, -(-int(c["ms"]) // 2048)), 0
    assert ssc._nat.lib().bcm_scan_bwd_workspace_bytes(a) > 0
    r1, g1 = _run_and_check(c, torch.float32, cuda_device)
    r2, g2 = _run_and_check(c, torch.float32, cuda_device)
    assert all(torch.equal(x, y) for x, y in zip(g1, g2))  # deterministic


@pytest.mark.parametrize("B,D,L,p,ps,N,dtype,markov,dim", [
    (64, 2, 1200, 0.6, 0.02, 16, torch.float32, False, None),  # split workgroups, 24-pass channels
    (64, 2, 1200, 0.6, 0.02, 64, torch.float32, False, None),  # four states per lane: 48-pass channels
    (40, 3, 900, 0.5, 0.02, 32, torch.float32, False, None),   # two states per lane, rounds not filled
    (64, 2, 1500, 0.5, 0.01, 16, torch.bfloat16, False, None),
    (48, 5, 1700, 0.0, 0.0, 16, torch.float32, True, None),    # Markov bursts: gaps past the decay table
    (48, 5, 1700, 0.0, 0.0, 64, torch.float32, True, None),
    (37, 4, 1300, 0.7, 0.03, 16, torch.float32, False, 5),     # 148 channels on 5 model channels (30 / 29 each)
])
def test_scan_bursty_ranked(cuda_device, B, D, L, p, ps, N, dtype, markov, dim):
    """Bursty streams with many channels per model channel: the state lanes
    rank the channels by length (the longest more than twice the mean) and
    split each model channel over workgroups. Parity against the oracle
    (forward, backward with and without the forward's state sums), Markov
    bursts with gaps past the decay table, a channel count that the model
    channels do not divide, and determinism."""
    print(f"bursty ranked case B={B} D={D} L={L} p={p}/{ps} N={N} {dtype} markov={markov} dim={dim}", flush=True)
    if markov:  # config 3's event law at a smaller size
        from bc_mamba_amd.workloads import _markov_events
        g = torch.Generator().manual_seed(B * L + N)
        mem = _markov_events(g, B * D, L).view(B, D, L).float()
        ch, t, k, cu, _, ms = orc.extract_base_events(mem.numpy(), 0.5)
        assert int(k.max()) > 256  # gaps past the decay table (computed decays)
        E = len(ch)
        c = dict(ch=ch, t=t, k=k, cu=cu, ms=ms, u=torch.randn(E, generator=g).to(dtype),
                 dout=torch.randn(E, generator=g).to(dtype), z=None,
                 dt_i=torch.nn.functional.softplus(torch.randn(D, generator=g) - 2.0),
                 dt_a=torch.nn.functional.softplus(torch.randn(D, generator=g) - 2.0),
                 A=-torch.exp(torch.rand(D, N, generator=g) * math.log(16.0)),
                 WB=torch.randn(D, N, generator=g) / math.sqrt(N), WC=torch.randn(D, N, generator=g) / math.sqrt(N),
                 D=torch.randn(D, generator=g))
    else:
        c = _case(B, D, L, p, N, dtype, seed=B + L + N, p_short=ps, dim=dim)
    NC, E, ms = B * D, len(c["ch"]), int(c["ms"])
    assert 2 * E < ms * NC  # bursty: the state lanes rank the channels
    _, g1 = _run_and_check(c, dtype, cuda_device)
    _run_and_check(c, dtype, cuda_device, use_acc=True)
    _, g2 = _run_and_check(c, dtype, cuda_device)
    assert all(torch.equal(x, y) for x, y in zip(g1, g2))  # deterministic


@pytest.mark.parametrize("N", [16, 64])
def test_scan_ranked_understated_max_seqlen(cuda_device, N):
    """A ranked, split backward under a max_seqlen of half the longest
    channel: every write stays inside the buffers sized from max_seqlen and
    the status word makes the entry point raise."""
    c = _case(64, 2, 1200, 0.6, N, torch.float32, seed=13, p_short=0.02, long_every=8)
    ms = int(c["ms"]) // 2
    NC, E = 128, len(c["ch"])
    assert 2 * E < ms * NC
    print(f"ranked seqlen status case: max_seqlen {ms} for channels of up to {int(c['ms'])} events", flush=True)
    dev = cuda_device
    cud = lambda x: x.to(dev)
    k_t, cu_t = torch.from_numpy(c["k"]).to(dev), torch.from_numpy(c["cu"]).to(dev)
    args = (cud(c["u"]), k_t, cu_t, ms, cud(c["dt_i"]), cud(c["dt_a"]), cud(c["A"]), cud(c["WB"]), cud(c["WC"]))
    x = torch.zeros((NC, ssc.n_chunks_for(ms), 2 * N), device=dev)
    with pytest.raises(RuntimeError, match="more than max_seqlen"):
        ssc.bwd_flat_ch(*args, cud(c["dout"]), x, D=cud(c["D"]), is_depthwise_bc=True)
    torch.cuda.synchronize()


@pytest.mark.parametrize("N", [16, 64])
@pytest.mark.parametrize("true_ms_scale", [3, 1])
def test_scan_reports_understated_max_seqlen(cuda_device, true_ms_scale, N):
    """A max_seqlen below the longest channel: the kernels keep every write
    inside the buffers sized from it and flag the channel in the status word;
    the Python entry points raise. With the true max_seqlen the status stays
    0 (regression test of the chunk_g bound and the status report)."""
    c = _case(2, 8, 1200, 0.4, N, torch.float32, seed=11, p_short=0.05)
    true_ms = int(c["ms"])
    ms = true_ms // true_ms_scale
    print(f"seqlen status case: max_seqlen {ms} for channels of up to {true_ms} events", flush=True)
    dev = cuda_device
    cud = lambda x: x.to(dev)
    k_t, cu_t = torch.from_numpy(c["k"]).to(dev), torch.from_numpy(c["cu"]).to(dev)
    args = (cud(c["u"]), k_t, cu_t, ms, cud(c["dt_i"]), cud(c["dt_a"]), cud(c["A"]), cud(c["WB"]), cud(c["WC"]))
    if ms < true_ms:
        with pytest.raises(RuntimeError, match="more than max_seqlen"):
            ssc.fwd_flat_ch(*args, D=cud(c["D"]), is_depthwise_bc=True)
        x = torch.zeros((16, ssc.n_chunks_for(ms), 2 * N), device=dev)
        with pytest.raises(RuntimeError, match="more than max_seqlen"):
            ssc.bwd_flat_ch(*args, cud(c["dout"]), x, D=cud(c["D"]), is_depthwise_bc=True)
    else:
        res = ssc.fwd_flat_ch(*args, D=cud(c["D"]), is_depthwise_bc=True)
        ssc.bwd_flat_ch(*args, cud(c["dout"]), res[1], D=cud(c["D"]), is_depthwise_bc=True)
    torch.cuda.synchronize()
