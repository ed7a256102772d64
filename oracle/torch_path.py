"""PyTorch restatement of BC_mamba's event path on the CPU - TEST
INFRASTRUCTURE ONLY (independent formulation for the oracle's tests and the
CPU baseline timed by bench.py). The product package never imports it.

Formulation (deliberately different from oracle/event_path.py):
  extract  comparison + torch.nonzero (extract_events_cuda.cu:192-312)
  gather   advanced indexing (e_model.py:196-201)
  scan     the textbook dense Mamba recurrence of selective_scan_ref
           (selective_scan_interface.py:708-774) on per-channel event
           streams padded to [NC, n_max] (padding is causal-inert), with
           variable B = u·W_B and C = u·W_C per event and D skip
  restore  torch.searchsorted forward fill (restore_dense_fwd_kernel.cuh:93-99)
  backward torch.autograd through all of the above
"""
import math

import torch

LOG2E = 1.4426950408889634


def extract(membrane, threshold):
    """-> ch, t, k, cu, counts (int64 tensors) for a [B, Dm, L] membrane."""
    B, Dm, L = membrane.shape
    NC = B * Dm
    mask = membrane.reshape(NC, L).float() > torch.tensor(float(threshold), dtype=torch.float32)
    ch, t = mask.nonzero(as_tuple=True)
    counts = mask.sum(1)
    cu = torch.zeros(NC + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(counts, 0)
    first = torch.ones_like(t, dtype=torch.bool)
    first[1:] = ch[1:] != ch[:-1]
    prev = torch.roll(t, 1)
    k = torch.where(first, t + 1, t - prev)
    return ch, t, k, cu, counts


def scan_dense(u, k, ch, cu, dt_idle, dt_active, A, W_B, W_C, D, clamp=True, dtype=torch.float32):
    """Dense selective_scan_ref form over padded event streams; differentiable
    in u and every parameter. Returns y per event (event order)."""
    NC = cu.numel() - 1
    dim, N = A.shape
    E = u.numel()
    pos = torch.arange(E) - cu[ch]
    nmax = int((cu[1:] - cu[:-1]).max()) if NC else 0
    dch = torch.arange(NC) % dim
    U = torch.zeros(NC, nmax, dtype=dtype).index_put((ch, pos), u.to(dtype))
    valid = torch.zeros(NC, nmax, dtype=torch.bool).index_put((ch, pos), torch.ones(E, dtype=torch.bool))
    Km1 = torch.zeros(NC, nmax, dtype=dtype).index_put((ch, pos), (k - 1).to(dtype))
    delta = dt_idle.to(dtype)[dch][:, None] * Km1 + dt_active.to(dtype)[dch][:, None]
    delta = torch.where(valid, delta, torch.zeros((), dtype=dtype))
    dA = delta[..., None] * A.to(dtype)[dch][:, None, :]
    deltaA = torch.exp2(torch.clamp(dA * LOG2E, -126.0, 126.0)) if clamp else torch.exp(dA)
    Bv = U[..., None] * W_B.to(dtype)[dch][:, None, :]
    Cv = U[..., None] * W_C.to(dtype)[dch][:, None, :]
    deltaB_u = delta[..., None] * U[..., None] * Bv
    h = torch.zeros(NC, N, dtype=dtype)
    ys = []
    for i in range(nmax):
        h = deltaA[:, i] * h + deltaB_u[:, i]
        ys.append((h * Cv[:, i]).sum(-1))
    y = torch.stack(ys, 1) if ys else torch.zeros(NC, 0, dtype=dtype)
    if D is not None:
        y = y + U * D.to(dtype)[dch][:, None]
    return y[ch, pos]


def restore(y, t, ch, cu, dim, L):
    """(B, L, dim) forward fill via searchsorted; differentiable in y."""
    NC = cu.numel() - 1
    E = y.numel()
    pos = torch.arange(E) - cu[ch]
    nmax = int((cu[1:] - cu[:-1]).max()) if NC else 0
    big = torch.iinfo(torch.int64).max
    T = torch.full((NC, max(nmax, 1)), big, dtype=torch.int64).index_put((ch, pos), t.to(torch.int64))
    Y = torch.zeros(NC, max(nmax, 1), dtype=y.dtype).index_put((ch, pos), y)
    q = torch.arange(L, dtype=torch.int64).expand(NC, L).contiguous()
    j = torch.searchsorted(T, q, right=True) - 1
    val = torch.where(j >= 0, Y.gather(1, j.clamp(min=0)), torch.zeros((), dtype=y.dtype))
    return val.reshape(NC // dim, dim, L).transpose(1, 2)


def path_fwd_bwd(membrane, x_conv, dout, threshold, dt_idle, dt_active, A, W_B, W_C, D):
    """One fwd+bwd of extract -> gather -> scan -> restore; returns
    (out (B,L,D), grads dict, E)."""
    x_conv = x_conv.detach().requires_grad_(True)
    params = [p.detach().requires_grad_(True) for p in (dt_idle, dt_active, A, W_B, W_C, D)]
    dti, dta, A_, WB, WC, D_ = params
    B, Dd, L = x_conv.shape
    ch, t, k, cu, _counts = extract(membrane, threshold)
    u = x_conv.reshape(B * Dd, L)[ch, t]
    y = scan_dense(u, k, ch, cu, dti, dta, A_, WB, WC, D_)
    out = restore(y, t, ch, cu, Dd, L)
    out.backward(dout)
    grads = dict(x_conv=x_conv.grad, dt_idle=dti.grad, dt_active=dta.grad, A=A_.grad, W_B=WB.grad, W_C=WC.grad,
                 D=D_.grad)
    return out.detach(), grads, int(ch.numel())


def n_chunks(max_seqlen):
    return max(1, math.ceil(int(max_seqlen) / 2048))
