"""Seeded synthetic workloads of the benchmark configurations (BASELINE.json
`configs`), generated on the CPU with torch.Generator in a fixed order and
then moved to the target device, so CPU and GPU see identical inputs.

  0  B=2  D=64  L=1024 N=16 fp32, membrane N(0,1) > 0.5 (~31% density)
  1  B=32 D=256 L=2048 N=16 fp32, i.i.d. Bernoulli(0.15) events   (headline)
  2  B=16 D=256 L=4096 N=16 bf16 u / dout (byte tokens -> embedding), 10%
  3  B=64 D=128 L=4000 N=64 fp32, two-state Markov bursts, half the
     channels forced below 2% density
  4  6-layer model (d_model 256, d_inner 512, N=16), L=1024, B=50, byte
     tokens: make_model_workload / SpikeMambaNet

Parameters: dt_idle, dt_active = softplus(N(0,1) - 2); A = -exp(U[ln 1, ln 16]);
W_B, W_C = N(0,1)/sqrt(N); D = 1. dout ~ N(0,1) of shape (B, L, D).
"""
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

__all__ = ["Workload", "make_workload", "CONFIGS", "SpikeMambaNet", "make_model_workload"]

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


# --------------------------------------------------------------- config 4
class _ResidualPreNorm(torch.nn.Module):
    """lra_impl.py:1381-1427 without the optional smoothness-loss terms:
    dv = core(s); v' = 0.95 v + dv; s' = core.to_spike(norm(v'))."""

    def __init__(self, d_model, core, leak_alpha=0.95):
        super().__init__()
        self.norm = torch.nn.LayerNorm(d_model)
        self.core = core
        self.leak_alpha = leak_alpha

    def forward(self, s_in, v_in):
        v_out = self.leak_alpha * v_in + self.core(s_in)
        return self.core.to_spike(self.norm(v_out)), v_out


class SpikeMambaNet(torch.nn.Module):
    """The config-4 model: SequenceClassifierBase of lra_impl.py:1429-1615
    with token input, sigmoid routing heads, STE spikes, LayerNorm, mean
    pooling and a spike-input head. in_prob and every block's prob_head get
    the bias logit(target_rate); in_prob's bias is frozen (:1490-1510). Each
    block's core is bc_mamba_amd.e_model.Mamba (spiking=False: the residual
    wrapper routes its output through to_spike)."""

    def __init__(self, d_model=256, n_layers=6, d_state=16, d_conv=4, expand=2, num_classes=10, vocab_size=256,
                 target_rate=0.3, routing_threshold=0.5):
        super().__init__()
        from .e_model import Mamba, SpikeSamplerSurrogate
        b = math.log(target_rate) - math.log(1.0 - target_rate)
        self.inp = torch.nn.Embedding(vocab_size, d_model)
        self.in_prob = torch.nn.Linear(d_model, d_model, bias=True)
        torch.nn.init.constant_(self.in_prob.bias, b)
        self.in_prob.bias.requires_grad_(False)
        self.in_spike = SpikeSamplerSurrogate(mode="ste", threshold=routing_threshold)
        blocks = []
        for i in range(n_layers):
            core = Mamba(d_model=d_model, d_state=d_state, d_conv=d_conv, expand=expand, spiking=False,
                         spike_mode="ste", prob_activation="sigmoid", threshold=routing_threshold, layer_idx=i)
            torch.nn.init.constant_(core.prob_head.bias, b)
            blocks.append(_ResidualPreNorm(d_model, core))
        self.blocks = torch.nn.ModuleList(blocks)
        self.norm = torch.nn.LayerNorm(d_model)
        self.head = torch.nn.Linear(d_model, num_classes)

    def forward(self, tokens):
        from . import projections
        v = self.inp(tokens.long())
        s = self.in_spike(torch.sigmoid(projections.linear(v, self.in_prob.weight, self.in_prob.bias)))
        for blk in self.blocks:
            s, v = blk(s, v)
        return self.head(self.norm(s).mean(dim=1))


def make_model_workload(seed=0, B=50, L=1024, device="cpu", **kw):
    """Config 4: the 6-layer model (random init from `seed`), byte tokens
    U{0..255} [B, L] and class labels, generated on the CPU."""
    torch.manual_seed(seed)
    model = SpikeMambaNet(**kw)
    g = torch.Generator().manual_seed(seed + 1)
    tokens = torch.randint(0, 256, (B, L), generator=g)
    labels = torch.randint(0, model.head.out_features, (B,), generator=g)
    return model.to(device), tokens.to(device), labels.to(device)
