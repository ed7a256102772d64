"""The Mamba block's token projections (in_proj, out_proj, prob_head of
e_model.py:258-506; in_prob of lra_impl.py:1490-1510) with a split-K weight
gradient.

A projection's weight gradient reduces over every token of the batch:
dW = dYᵀ X with B·L = 51 200 rows at config 4 and a small [out, in] result.
For [256, 51200] @ [51200, 512] hipBLASLt picks a tile of 32 x 256 and ~40
workgroups on a 256-CU MI355X: 563 µs, 24 TFLOP/s. Splitting the tokens into
8 chunks gives one batched product with 8x the workgroups and a fixed-order
sum of the 8 partials: ~118 µs (the sum adds a few µs), deterministic, fp32
throughout. The forward calls and the input gradients are the same
products as before; only the weight gradient's summation order changes
(fp32 rounding, ~4e-6 relative).

Used for fp32 tensors with at least 8192 tokens divisible by the split;
anything else takes the plain product.
"""
import torch
import torch.nn.functional as F

__all__ = ["linear", "proj_tokens_last", "weight_grad"]

SPLIT = 8
MIN_TOKENS = 8192


def _split_ok(m, *ts):
    return m >= MIN_TOKENS and m % SPLIT == 0 and all(t.dtype == torch.float32 for t in ts)


def weight_grad(g, x, tokens_first=True):
    """Σ over tokens of g ⊗ x: gᵀ @ x for g [M, N] (tokens_first) or g @ x
    for g [N, M], with x [M, K]. Chunks of M/SPLIT tokens, one batched
    product, the partials summed in chunk order."""
    m = x.size(0)
    if not _split_ok(m, g, x):
        return g.t() @ x if tokens_first else g @ x
    c = m // SPLIT
    if tokens_first:
        gs = g.reshape(SPLIT, c, g.size(1)).transpose(1, 2)  # [S, N, c]
    else:
        gs = g.reshape(g.size(0), SPLIT, c).transpose(0, 1)  # [S, N, c]
    return torch.bmm(gs, x.reshape(SPLIT, c, x.size(1))).sum(0)


class _LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return F.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, gy):
        x, weight = ctx.saved_tensors
        g2 = gy.reshape(-1, gy.size(-1))
        dx = (g2 @ weight).view(x.shape) if ctx.needs_input_grad[0] else None
        dw = weight_grad(g2, x.reshape(-1, x.size(-1))) if ctx.needs_input_grad[1] else None
        db = g2.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return dx, dw, db


def linear(x, weight, bias=None):
    """F.linear(x, weight, bias) with the split-K weight gradient."""
    return _LinearFn.apply(x, weight, bias)


class _ProjTokensLastFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, weight, h2d):
        ctx.save_for_backward(weight, h2d)
        return weight @ h2d.t()

    @staticmethod
    def backward(ctx, g):
        weight, h2d = ctx.saved_tensors
        dw = weight_grad(g, h2d, tokens_first=False) if ctx.needs_input_grad[0] else None
        dh = g.t() @ weight if ctx.needs_input_grad[1] else None
        return dw, dh


def proj_tokens_last(weight, h2d):
    """weight @ h2dᵀ ([out, M] from weight [out, in] and tokens h2d [M, in]:
    the block's `in_proj.weight @ rearrange(h, "b l d -> d (b l)")`) with the
    split-K weight gradient."""
    return _ProjTokensLastFn.apply(weight, h2d)
