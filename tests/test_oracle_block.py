"""The float64 block composition of oracle/block.py (the checker of the
fused Mamba block) against an independent formulation: the same dense
parts with the event path of oracle/torch_path.py (padded textbook scan,
searchsorted restore) differentiated by torch autograd. Output and every
parameter and input gradient must agree to float64 rounding, so a wrong
gradient slot, a transposed operand or a dropped term in the oracle node's
backward fails here."""
import numpy as np
import torch

from bc_mamba_amd import e_model
from oracle import block as ob
from oracle import torch_path as tp


def _torch_event_path(xc, dt_idle, dt_active, A, W_B, W_C, D, events):
    ch, t, k, cu, _ = events
    ch, t, k, cu = (torch.from_numpy(np.asarray(v, np.int64)) for v in (ch, t, k, cu))
    B, Din, L = xc.shape
    u = xc.reshape(B * Din, L)[ch, t]
    y = tp.scan_dense(u, k, ch, cu, dt_idle, dt_active, A, W_B, W_C, D, dtype=torch.float64)
    return tp.restore(y, t, ch, cu, Din, L)


def test_oracle_block_matches_autograd_formulation():
    torch.manual_seed(0)
    blk = e_model.Mamba(d_model=8, d_state=4, expand=2, device="cpu")
    with torch.no_grad():  # non-trivial values for every parameter
        blk.D.uniform_(0.5, 1.5)
        blk.W_BC.normal_(0.0, 0.5)
        blk.conv1d.bias.normal_(0.0, 0.2)
    v = torch.randn(2, 40, 8, dtype=torch.float64, requires_grad=True)
    g = torch.randn(2, 40, 8, dtype=torch.float64)
    res = []
    for path in (None, _torch_event_path):
        vv = v.detach().clone().requires_grad_(True)
        p = ob.params_of(blk)
        s, prob = ob.spike_head(blk, vv, p)
        out, p = ob.mamba_forward(blk, s, p=p, event_path=path)
        out.backward(g)
        res.append((out.detach(), vv.grad, {n: q.grad for n, q in p.items()}))
    (o1, dv1, g1), (o2, dv2, g2) = res
    assert ob.block_events(s.detach().numpy(), blk.threshold, 2)[0].size > 50
    np.testing.assert_allclose(o1.numpy(), o2.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dv1.numpy(), dv2.numpy(), rtol=1e-9, atol=1e-12)
    assert g1.keys() == g2.keys() and len(g1) >= 10
    for n in g1:
        assert g1[n] is not None and g2[n] is not None, n
        np.testing.assert_allclose(g1[n].numpy(), g2[n].numpy(), rtol=1e-9, atol=1e-12, err_msg=n)
