"""Seeded synthetic workloads of the benchmark configurations (BASELINE.json
`configs`), generated on the CPU with torch.Generator in a fixed order and
then moved to the target device, so CPU and GPU see identical inputs.

  0  B=2  D=64  L=1024 N=16 fp32, membrane N(0,1) > 0.5 (~31% density)
  1  B=32 D=256 L=2048 N=16 fp32, i.i.d. Bernoulli(0.15) events   (headline)
  2  B=16 D=256 L=4096 N=16 bf16 u / dout (byte tokens -> embedding), 10%
  3  B=64 D=128 L=4000 N=64 fp32, two-state Markov bursts, half the
     channels forced below 2% density

Parameters: dt_idle, dt_active = softplus(N(0,1) - 2); A = -exp(U[ln 1, ln 16]);
W_B, W_C = N(0,1)/sqrt(N); D = 1. dout ~ N(0,1) of shape (B, L, D).
"""
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

__all__ = ["Workload", "make_workload", "CONFIGS"]

CONFIGS = {
    0: dict(B=2, D=64, L=1024, N=16, dtype=torch.float32, events="gauss"),
    1: dict(B=32, D=256, L=2048, N=16, dtype=torch.float32, events="bernoulli", p=0.15),
    2: dict(B=16, D=256, L=4096, N=16, dtype=torch.bfloat16, events="bernoulli", p=0.10, tokens=True),
    3: dict(B=64, D=128, L=4000, N=64, dtype=torch.float32, events="markov"),
}


@dataclass
class Workload:
    cfg: int
    B: int
    D: int
    L: int
    N: int
    dtype: torch.dtype
    threshold: float
    membrane: torch.Tensor  # (B, D, L) float32, compared against threshold
    x_conv: torch.Tensor    # (B, D, L) dtype, gathered at the events -> u
    dt_idle: torch.Tensor
    dt_active: torch.Tensor
    A: torch.Tensor
    W_B: torch.Tensor
    W_C: torch.Tensor
    D_skip: torch.Tensor
    dout: torch.Tensor      # (B, L, D) dtype

    def to(self, device):
        kw = {f: getattr(self, f) for f in self.__dataclass_fields__}
        for f, v in kw.items():
            if isinstance(v, torch.Tensor):
                kw[f] = v.to(device)
        return Workload(**kw)


def _markov_events(g, NC, L):
    """Two-state chain per channel: on->on 0.9, off->off 0.98, start drawn
    from the stationary law (on = 0.02 / 0.12); a seeded half of the channels
    is replaced by Bernoulli(0.015)."""
    p_on = 0.02 / (0.1 + 0.02)
    state = torch.rand(NC, generator=g) < p_on
    u = torch.rand(NC, L, generator=g)
    ev = torch.empty(NC, L, dtype=torch.bool)
    for t in range(L):
        stay = torch.where(state, u[:, t] < 0.9, u[:, t] < 0.98)
        state = torch.where(stay, state, ~state)
        ev[:, t] = state
    sparse = torch.randperm(NC, generator=g)[: NC // 2]
    ev[sparse] = torch.rand(NC // 2, L, generator=g) < 0.015
    return ev


def make_workload(cfg, seed=0, device="cpu", B=None, D=None, L=None, N=None):
    """Build config `cfg` (optionally with overridden sizes for tests)."""
    c = dict(CONFIGS[cfg])
    B = c["B"] if B is None else B
    D = c["D"] if D is None else D
    L = c["L"] if L is None else L
    N = c["N"] if N is None else N
    dtype = c["dtype"]
    g = torch.Generator().manual_seed(seed)
    if c["events"] == "gauss":
        membrane = torch.randn(B, D, L, generator=g)
    elif c["events"] == "bernoulli":
        membrane = (torch.rand(B, D, L, generator=g) < c["p"]).float()
    else:
        membrane = _markov_events(g, B * D, L).view(B, D, L).float()
    if c.get("tokens"):
        tokens = torch.randint(0, 256, (B, L), generator=g)
        emb = torch.randn(256, D, generator=g)
        x_conv = emb[tokens].transpose(1, 2).contiguous().to(dtype)
    else:
        x_conv = torch.randn(B, D, L, generator=g).to(dtype)
    dt_idle = F.softplus(torch.randn(D, generator=g) - 2.0)
    dt_active = F.softplus(torch.randn(D, generator=g) - 2.0)
    A = -torch.exp(torch.rand(D, N, generator=g) * math.log(16.0))
    W_B = torch.randn(D, N, generator=g) / math.sqrt(N)
    W_C = torch.randn(D, N, generator=g) / math.sqrt(N)
    D_skip = torch.ones(D)
    dout = torch.randn(B, L, D, generator=g).to(dtype)
    w = Workload(cfg, B, D, L, N, dtype, 0.5, membrane, x_conv, dt_idle, dt_active, A, W_B, W_C, D_skip, dout)
    return w if device == "cpu" else w.to(device)
