"""Drop-in for `causal_conv1d_fn`, the causal depthwise conv1d the
reference's Mamba block calls when the causal_conv1d package is importable
(e_model.py:442-451; otherwise it runs nn.Conv1d(groups=d_inner,
padding=d_conv-1) and SiLU, the same function). Backed by the HIP kernels
bcm_causal_conv1d_fwd / _bwd of libbcm_event_scan.so.

    causal_conv1d_fn(x [B, D, L], weight [D, K], bias [D] or None,
                     activation None | "silu" | "swish") -> [B, D, L]

The package's sequence-index, initial-state and final-state arguments are
not part of the path and must be left at their defaults.
"""
import torch

try:
    from . import _native as _nat
except ImportError:  # imported with this directory on sys.path
    import _native as _nat

__all__ = ["causal_conv1d_fn", "CausalConv1dFn", "conv1d_bwd_events"]


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


class CausalConv1dFn(torch.autograd.Function):
    """out = act(bias + sum_k w[:, k] x[..., t-(K-1)+k]) with x = 0 before t=0;
    backward gives dx, dweight [D, K] and dbias (fp32 weights)."""

    @staticmethod
    def forward(ctx, x, weight, bias, silu: bool):
        x = x.contiguous()
        w = weight.contiguous().float()
        b = bias.contiguous().float() if bias is not None else None
        B, D, L = x.shape
        out = torch.empty_like(x)
        with torch.cuda.device(x.device):
            _nat.call("bcm_causal_conv1d_fwd", x.data_ptr(), _nat.dtype_code(x.dtype), w.data_ptr(),
                      b.data_ptr() if b is not None else None, B, D, L, int(w.size(1)), int(silu), out.data_ptr(),
                      _nat.stream_of(x))
        ctx.save_for_backward(x, w, b)
        ctx.silu, ctx.has_bias, ctx.wdtype = silu, bias is not None, weight.dtype
        return out

    @staticmethod
    def backward(ctx, dout):
        x, w, b = ctx.saved_tensors
        dout = dout.contiguous()
        B, D, L = x.shape
        dx = torch.empty_like(x)
        dw = torch.empty_like(w)
        db = torch.empty(D, dtype=torch.float32, device=x.device) if ctx.has_bias else None
        K = int(w.size(1))
        with torch.cuda.device(x.device):
            nbytes = int(_nat.lib().bcm_causal_conv1d_bwd_workspace_bytes(B, D, L, K))
            ws = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=x.device) if nbytes else None
            _nat.call("bcm_causal_conv1d_bwd", x.data_ptr(), _nat.dtype_code(x.dtype), w.data_ptr(),
                      b.data_ptr() if b is not None else None, dout.data_ptr(), B, D, L, K,
                      int(ctx.silu), dx.data_ptr(), dw.data_ptr(), db.data_ptr() if db is not None else None,
                      ws.data_ptr() if ws is not None else None, nbytes, _nat.stream_of(x))
        return dx, dw.to(ctx.wdtype), (db.to(ctx.wdtype) if db is not None else None), None


def conv1d_bwd_events(x, weight, bias, silu, du, event_index):
    """Backward of the conv evaluated at the events (extract_events_indexed
    with conv=...) and the gather, from du [E] (the gradient of x_events):
    (dx with x's strides, dweight [D, K] fp32, dbias [D] fp32 or None)
    (bcm_causal_conv1d_bwd_events). No reference counterpart as one call:
    it is GatherEventsFn.backward followed by the conv backward."""
    B, D, L = x.shape
    bitmask, tile_start, mrd = event_index
    w = weight.detach().float().contiguous()
    b = bias.detach().float().contiguous() if bias is not None else None
    _check(du.dtype == x.dtype and du.is_contiguous(), "conv1d_bwd_events: du must be contiguous, x's dtype")
    dx = torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device=x.device)
    dw = torch.empty_like(w)
    db = torch.empty(D, dtype=torch.float32, device=x.device) if bias is not None else None
    K = int(w.size(1))
    with torch.cuda.device(x.device):
        nbytes = int(_nat.lib().bcm_causal_conv1d_bwd_events_workspace_bytes(B, D, K))
        ws = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=x.device)
        _nat.call("bcm_causal_conv1d_bwd_events", x.data_ptr(), _nat.dtype_code(x.dtype), x.stride(0), x.stride(1),
                  B, D, L, w.data_ptr(), b.data_ptr() if b is not None else None, K, int(bool(silu)),
                  du.data_ptr(), int(du.numel()), bitmask.data_ptr(), int(mrd), tile_start.data_ptr(),
                  dx.data_ptr(), dw.data_ptr(), db.data_ptr() if db is not None else None, ws.data_ptr(), nbytes,
                  _nat.stream_of(x))
    return dx, dw, db


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None, return_final_states=False,
                     final_states_out=None, activation=None):
    """x [B, D, L] (fp32/fp16/bf16, CUDA), weight [D, K] (K <= 8), bias [D]."""
    fn = "causal_conv1d_fn"
    _check(activation in (None, "silu", "swish"), f"{fn}: activation must be None, silu or swish")
    _check(seq_idx is None and initial_states is None and not return_final_states and final_states_out is None,
           f"{fn}: seq_idx / initial_states / final states are not supported by the MI355X build")
    _check(x.is_cuda and weight.is_cuda and (bias is None or bias.is_cuda), f"{fn}: tensors must be on the GPU")
    _check(x.dim() == 3, f"{fn}: x must be [batch, dim, seqlen]")
    _check(weight.dim() == 2 and weight.size(0) == x.size(1), f"{fn}: weight must be [dim, width]")
    _check(1 <= weight.size(1) <= 8, f"{fn}: width must be in [1, 8]")
    _check(bias is None or tuple(bias.shape) == (x.size(1),), f"{fn}: bias must be [dim]")
    _check(x.dtype in (torch.float32, torch.float16, torch.bfloat16), f"{fn}: x must be fp32/fp16/bf16")
    return CausalConv1dFn.apply(x, weight, bias, activation in ("silu", "swish"))
