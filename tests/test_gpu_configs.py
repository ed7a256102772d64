"""BASELINE configurations 1-3 at full size, in the kernel forms bench.py
times (bc_mamba_amd.fused_step.FusedStep: count with block sums, the fill
deriving its offsets and gathering x_conv at the events without ch / t
streams, the indexed restore, the scan backward writing the dense dx rows),
every output compared with the float64 oracle:

  indices  k, cu_seqlens, max_seqlen, the tile table: bit-exact
  gather   u = x_conv at the events: bit-exact
  restore  out (from the GPU's y): bit-exact (a copy); dy: fp32 bar
  scan     y, x, du and the six parameter gradients: rtol 1e-4 (fp32) or
           2e-2 (bf16 outputs), absolute floor 1e-6 * max|ref|
  gather backward  dx = du at the events, 0 elsewhere: bit-exact

Each stage is fed the GPU's own inputs (so each comparison isolates one
kernel) and the end-to-end restore output is also compared with the pure
oracle chain. Reference contract: selective_scan.cpp:674-1153,
restore_dense.cpp:43-202, extract_events_cuda.cu:192-418.
"""
import numpy as np
import pytest
import torch

from bc_mamba_amd.fused_step import FusedStep
from bc_mamba_amd.workloads import make_workload
from conftest import assert_close
from oracle import event_path as orc

pytestmark = pytest.mark.gpu

FLOOR = 1e-6  # absolute floor of the fp32 bar, relative to max|ref|


def tile_table(ch, t, NC, L):
    """Oracle tile table [NC, ceil(L/64)+1]: the index of each channel's
    first event at or after step 64j (the channel's end for j = ntiles)."""
    nT = (L + 63) // 64
    key = ch.astype(np.int64) * L + t
    j = np.minimum(np.arange(nT + 1) * 64, L)
    q = np.arange(NC, dtype=np.int64)[:, None] * L + j[None, :]
    return np.searchsorted(key, q.ravel(), side="left").reshape(NC, nT + 1).astype(np.int32)


def n(v):
    return v.detach().float().cpu().numpy()


def run_step(cfg, dev, **kw):
    w = make_workload(cfg, **kw)
    print(f"config {cfg} {kw}: B={w.B} D={w.D} L={w.L} N={w.N} {w.dtype}", flush=True)
    wd = w.to(dev)
    st = FusedStep(wd, dev)
    st.step()
    torch.cuda.synchronize()
    return w, st


def check_indices(w, st):
    NC, L = w.B * w.D, w.L
    och, ot, ok, ocu, ocounts, oms = orc.extract_base_events(w.membrane.numpy(), w.threshold)
    assert st.E == len(och) and st.ms == oms
    assert np.array_equal(st.k.cpu().numpy(), ok), "k"
    assert np.array_equal(st.cu.cpu().numpy(), ocu), "cu_seqlens"
    assert np.array_equal(st.tile_start.cpu().numpy(), tile_table(och, ot, NC, L)), "tile table"
    u = st.u.cpu()
    assert torch.equal(u, w.x_conv.reshape(NC, L)[torch.from_numpy(och).long(), torch.from_numpy(ot).long()]), "u"
    return och, ot, ok, ocu, oms


def check_restore(w, st, och, ot, ocu, sel=None):
    """Restore forward from the GPU's y (a copy: bit-exact) and restore
    backward (fp32 sums, stored in fp32 or in u's 16-bit dtype) against the
    oracle, on batches `sel` (all if None)."""
    B, D, L = w.B, w.D, w.L
    bs = range(B) if sel is None else sel
    y = st.y.float().cpu().numpy()
    dy = st.dy_restore.float().cpu().numpy()
    # a 16-bit dy is the fp32 sum rounded once: within half an ulp of bf16
    dy_rtol = 1e-4 if st.dy_restore.dtype == torch.float32 else 2.0 ** -8 + 1e-4
    dense = st.dense.float().cpu().numpy()
    dout = w.dout.float().numpy()
    for b in ([None] if sel is None else bs):
        c0, c1 = (0, B * D) if b is None else (b * D, (b + 1) * D)
        e0, e1 = int(ocu[c0]), int(ocu[c1])
        cu_s = (ocu[c0:c1 + 1] - e0).astype(np.int32)
        rows = slice(None) if b is None else slice(b, b + 1)
        ref = orc.restore_fwd(y[e0:e1], ot[e0:e1], cu_s, D, L)
        assert np.array_equal(dense[rows], ref.astype(np.float32)), f"restore out (batch {b})"
        ref_dy = orc.restore_bwd(dout[rows], ot[e0:e1], cu_s, D, L)
        assert_close(dy[e0:e1], ref_dy, dy_rtol, FLOOR, f"restore dy (batch {b})")


def scan_oracle(w, st, ocu, oms, c0, c1):
    """Oracle forward and backward of channels [c0, c1) on the GPU's u and
    dout (dout in the dtype the scan read it)."""
    e0, e1 = int(ocu[c0]), int(ocu[c1])
    cu_s = (ocu[c0:c1 + 1] - e0).astype(np.int32)
    D = w.D
    assert c0 % D == 0 and (c1 - c0) % D == 0  # whole batches: model channel d = ch % D holds
    P = [n(v) for v in (w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C)]
    u = n(st.u)[e0:e1]
    k = st.k.cpu().numpy()[e0:e1]
    dout = n(st.dy_buf[:st.E])[e0:e1]
    y, x = orc.scan_fwd(u, k, cu_s, oms, *P, n(w.D_skip))
    g = orc.scan_bwd(u, k, cu_s, oms, *P, dout, n(w.D_skip))
    return (e0, e1), y, x, g


def check_scan_channels(w, st, ocu, oms, och, ot, c0, c1, rtol_out, ref=None):
    """Scan out, x, du and the dense dx rows of channels [c0, c1) against
    the oracle (`ref`: scan_oracle's result for them, if already run)."""
    (e0, e1), y, x, g = ref if ref is not None else scan_oracle(w, st, ocu, oms, c0, c1)
    assert_close(n(st.y)[e0:e1], y, rtol_out, FLOOR, f"scan out [{c0},{c1})")
    assert_close(n(st.xs)[c0:c1], x, 1e-4, FLOOR, f"scan x [{c0},{c1})")
    assert_close(n(st.du)[e0:e1], g[0], rtol_out, FLOOR, f"du [{c0},{c1})")
    # gather backward rows: du at the events, 0 elsewhere (bit-exact)
    L = w.L
    dx = st.dx.reshape(-1, L)[c0:c1].cpu()
    ref = torch.zeros(c1 - c0, L, dtype=st.dx.dtype)
    ref[torch.from_numpy(och[e0:e1] - c0).long(), torch.from_numpy(ot[e0:e1]).long()] = st.du[e0:e1].cpu()
    assert torch.equal(dx, ref), f"dx rows [{c0},{c1})"
    return g


def check_param_grads(st, grads_ref, rtol=1e-4):
    names = ("dA", "dW_B", "dW_C", "ddt_idle", "ddt_active", "dD")
    for name, got, ref in zip(names, st.grads, grads_ref):
        assert_close(n(got), ref, rtol, FLOOR, name)


@pytest.mark.parametrize("cfg", [1, 2])
def test_config_full_size_bench_kernels(cuda_device, cfg, scan_kernel):
    """Configs 1 (fp32, 15 %) and 2 (bf16 u / out / dout, token embedding,
    L 4096, 10 %): the whole step at full size, every channel, under both
    dstate-16 scan families."""
    w, st = run_step(cfg, cuda_device)
    och, ot, ok, ocu, oms = check_indices(w, st)
    check_restore(w, st, och, ot, ocu)
    rtol = 1e-4 if w.dtype == torch.float32 else 2e-2
    g = check_scan_channels(w, st, ocu, oms, och, ot, 0, w.B * w.D, rtol)
    check_param_grads(st, g[1:7])
    # end to end: the pure oracle chain from the membrane to the restore output
    P = [n(v) for v in (w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C)]
    u = orc.gather_fwd(w.x_conv.float().numpy(), och, ot)
    y, _ = orc.scan_fwd(u, ok, ocu, oms, *P, n(w.D_skip))
    ref = orc.restore_fwd(y, ot, ocu, w.D, w.L)
    assert_close(n(st.dense), ref, rtol, FLOOR, "end-to-end restore out")


def test_config3_full_size_bench_kernels(cuda_device):
    """Config 3 (B64 D128 L4000 N64, bursty Markov events with half the
    channels below 2 %): multi-pass channels with chunk_g, model channels
    split over workgroups. Everything on every channel of all 64 batches:
    indices on the full membrane, restore out and dy, and the oracle run in
    8-batch slices for scan out, x, du, the dense dx rows and the six
    parameter gradients (the slices' partial sums added)."""
    w, st = run_step(3, cuda_device)
    assert st.chunk_g is not None and st.split_ws is not None  # the multi-pass and split forms run
    och, ot, ok, ocu, oms = check_indices(w, st)
    B, D = w.B, w.D
    check_restore(w, st, och, ot, ocu)
    acc = None
    for b0 in range(0, B, 8):
        c0, c1 = b0 * D, (b0 + 8) * D
        print(f"config 3: batches {b0}..{b0 + 7}", flush=True)
        g = check_scan_channels(w, st, ocu, oms, och, ot, c0, c1, 1e-4, ref=scan_oracle(w, st, ocu, oms, c0, c1))
        part = g[1:7]
        acc = list(part) if acc is None else [a + p for a, p in zip(acc, part)]
    check_param_grads(st, acc)
