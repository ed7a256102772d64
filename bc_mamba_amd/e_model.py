"""Drop-in for the event-path pieces of the reference's spike_mamba/e_model.py:
`RestoreDenseFn` / `restore_dense_fn` (:123-161), `GatherEventsFn` (:167-193),
`TwoLevelDelta` (:210-230), `SpikeSamplerSurrogate` (:233-254) and the
`Mamba` block (:258-506) with `extract_events_1d` (:361-409).

The block runs the same composition as the reference: dense in_proj GEMM,
depthwise causal conv + SiLU, then the event path on the HIP
kernels (extraction, gather, flat selective scan, zero-order-hold restore),
then out_proj. With `fused_event_path=True` (default) the block calls the
fused entry points: one extraction pass that also gathers x_conv at the
events and builds the event index, the restore reads that index instead of
rebuilding it, the scan backward writes the dense x_conv gradient rows from
the same index (no separate gather backward), and the per-block host syncs
drop from two to one. The fused path's token projections (in_proj, out_proj,
prob_head) take their weight gradients as split-K products
(`projections`). With `conv_at_events=True` (default) the depthwise
conv + SiLU is evaluated only at the events, by the extraction itself, and
its backward goes from du straight to the conv input's gradient: no dense
x_conv exists in either direction. With `fused_out_proj=True` (default; fp32)
the restore and out_proj run as one op reading the event index: the dense
restore output is not kept for the backward and its gradient is never
formed (the input gradient of out_proj and the restore backward are one
kernel); `fused_out_proj="mfma"` also runs the forward and the weight
gradient as this package's matrix-core kernels, with no dense restore output
at all. Results match the unfused composition
(forward values identical; the conv weight gradients up to summation
order).

The decode `step` / inference cache of the reference are not part of the
event path (the reference's own `step` reads an undefined `self.pw_B`).
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F
from einops import rearrange, repeat

try:
    from . import _native as _nat
    from . import extract_events_cuda as _ee_cuda
    from . import restore_dense_cuda_nodecay
    from . import projections
    from . import selective_scan_cuda
    from .causal_conv1d import causal_conv1d_fn, conv1d_bwd_events
    from .runtime_breakdown import cuda_stage
    from .selective_scan_interface import selective_scan_flat_ch_fn
except ImportError:  # imported with this directory on sys.path
    import _native as _nat
    import extract_events_cuda as _ee_cuda
    import restore_dense_cuda_nodecay
    import projections
    import selective_scan_cuda
    from causal_conv1d import causal_conv1d_fn, conv1d_bwd_events
    from runtime_breakdown import cuda_stage
    from selective_scan_interface import selective_scan_flat_ch_fn

_HAS_EE_CUDA = True
_HAS_GATHER_CUDA = True


class RestoreDenseFn(torch.autograd.Function):
    """Zero-order-hold restore. forward(y_flat, time_steps_i32, cu_seqlens,
    dim, seqlen) -> (B, L, D); backward -> (dy_flat, None, None, None, None)."""

    @staticmethod
    def forward(ctx, y_flat, time_steps_i32, cu_seqlens, dim: int, seqlen: int):
        out = restore_dense_cuda_nodecay.restore_dense_fwd(y_flat, time_steps_i32, cu_seqlens, dim, seqlen)
        ctx.save_for_backward(time_steps_i32, cu_seqlens)
        ctx.dim, ctx.seqlen = dim, seqlen
        return out

    @staticmethod
    def backward(ctx, dout):
        time_steps_i32, cu_seqlens = ctx.saved_tensors
        with cuda_stage("restore_backward"):
            dy = restore_dense_cuda_nodecay.restore_dense_bwd(dout.contiguous(), time_steps_i32, cu_seqlens,
                                                              ctx.dim, ctx.seqlen)
        return dy, None, None, None, None


def restore_dense_fn(y_flat, time_steps_i32, cu_seqlens, dim: int, seqlen: int):
    return RestoreDenseFn.apply(y_flat, time_steps_i32, cu_seqlens, dim, seqlen)


class GatherEventsFn(torch.autograd.Function):
    """Differentiable gather of x_conv [B, D, L] at (channel_ids, time_steps);
    backward scatters into a dense zero tensor."""

    @staticmethod
    def forward(ctx, x_conv, channel_ids_i32, time_steps_i32):
        x_c = x_conv.contiguous()
        out_x = _ee_cuda.gather_events_fwd(x_c, channel_ids_i32, time_steps_i32)[0]
        ctx.save_for_backward(channel_ids_i32, time_steps_i32)
        ctx.shape = x_c.shape
        return out_x

    @staticmethod
    def backward(ctx, grad_x):
        channel_ids_i32, time_steps_i32 = ctx.saved_tensors
        B, D, L = ctx.shape
        with cuda_stage("gather_scatter_backward"):
            dx_flat = _ee_cuda.gather_events_bwd(grad_x.contiguous(), channel_ids_i32, time_steps_i32, B * D, L)[0]
        return dx_flat.view(B, D, L), None, None


def _gather_events_cuda(x_conv, channel_ids_i32, time_steps_i32):
    return GatherEventsFn.apply(x_conv, channel_ids_i32, time_steps_i32)


_gather_events_fn = _gather_events_cuda


class _IndexedGatherFn(torch.autograd.Function):
    """x_conv values already gathered by the fused extraction; the backward
    writes the dense gradient row by row from the event index."""

    @staticmethod
    def forward(ctx, x_conv, payload, event_index):
        # payload = (x_events,): kept out of the autograd inputs on purpose
        ctx.event_index = event_index
        ctx.shape = x_conv.shape
        return payload[0]

    @staticmethod
    def backward(ctx, grad_x):
        B, D, L = ctx.shape
        bitmask, tile_start, expand = ctx.event_index
        g = grad_x.contiguous()
        dx = torch.empty((B, D, L), dtype=g.dtype, device=g.device)
        with cuda_stage("gather_scatter_backward"):
            _nat.call("bcm_gather_bwd_rows", _nat.ptr(g), _nat.dtype_code(g.dtype), _nat.ptr(bitmask), int(expand),
                      _nat.ptr(tile_start), B * D, L, _nat.ptr(dx), _nat.stream_of(g))
        return dx, None, None


def _event_scan_fwd(ctx, x_ev, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, W_B, W_C, D):
    """Depthwise flat scan forward of the fused block. Returns (out, the
    tensors the backward reads), for ctx.save_for_backward."""
    dt_idle, dt_active = dt_idle.contiguous(), dt_active.contiguous()
    A, W_B, W_C = A.contiguous(), W_B.contiguous(), W_C.contiguous()
    chunk_g = selective_scan_cuda.chunk_states_buffer(x_ev, cu_seqlens, max_seqlen, A)
    acc = torch.empty(x_ev.shape, dtype=torch.float32, device=x_ev.device)  # per-event state sums
    out, xs = selective_scan_cuda.fwd_flat_ch(x_ev, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, W_B, W_C, D,
                                              None, is_depthwise_bc=True, _chunk_g=chunk_g, _trusted_seqlen=True,
                                              _acc=acc)
    ctx.chunk_g, ctx.acc, ctx.max_seqlen, ctx.has_D = chunk_g, acc, max_seqlen, D is not None
    return out, [x_ev, k_flat, cu_seqlens, dt_idle, dt_active, A, W_B, W_C, xs] + ([D] if D is not None else [])


def _event_scan_bwd(ctx, saved, dout, rows=None):
    """(du, dt_idle, dt_active, dA, dW_B, dW_C, dD) of the fused block's scan
    from the tensors _event_scan_fwd saved; with rows = (bitmask, expand,
    tile_start, dx) the scan kernel also writes the dense gather backward
    into dx, and du (which then has no other use) is None where that kernel
    writes the rows itself."""
    x_ev, k_flat, cu_seqlens, dt_idle, dt_active, A, W_B, W_C, xs = saved[:9]
    D = saved[9] if ctx.has_D else None
    res = selective_scan_cuda.bwd_flat_ch(x_ev, k_flat, cu_seqlens, ctx.max_seqlen, dt_idle, dt_active, A, W_B, W_C,
                                          dout.contiguous(), xs, D, is_depthwise_bc=True, _chunk_g=ctx.chunk_g,
                                          _rows=rows, _trusted_seqlen=True, _acc=ctx.acc,
                                          _discard_du=rows is not None)
    du, dA, dW_B, dW_C, ddt_idle, ddt_active = res[:6]
    return du, ddt_idle, ddt_active, dA, dW_B, dW_C, (res[6] if D is not None else None)


class _IndexedScanFn(torch.autograd.Function):
    """The gather of x_conv at the events (already done by the fused
    extraction) and the depthwise flat scan as one autograd node. Its
    backward writes the dense x_conv gradient from the scan kernel
    (bcm_scan_bwd_rows) instead of scattering du in a second pass. Same
    results as _IndexedGatherFn followed by SelectiveScanFlatChFn."""

    @staticmethod
    def forward(ctx, x_conv, payload, event_index, k_flat, cu_seqlens, max_seqlen: int, dt_idle, dt_active, A, W_B,
                W_C, D):
        # payload = (x_events,): kept out of the autograd inputs on purpose
        ctx.event_index, ctx.shape = event_index, x_conv.shape
        out, saved = _event_scan_fwd(ctx, payload[0], k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, W_B,
                                     W_C, D)
        ctx.save_for_backward(*saved)
        return out

    @staticmethod
    def backward(ctx, dout):
        B, Dm, L = ctx.shape
        bitmask, tile_start, expand = ctx.event_index
        saved = ctx.saved_tensors
        x_ev = saved[0]
        dx = torch.empty((B * Dm, L), dtype=x_ev.dtype, device=x_ev.device)
        with cuda_stage("sparse_scan_backward"):
            _du, *grads = _event_scan_bwd(ctx, saved, dout, rows=(bitmask, expand, tile_start, dx))
        return (dx.view(B, Dm, L), None, None, None, None, None, *grads)


class _IndexedConvScanFn(torch.autograd.Function):
    """The block's depthwise causal conv + SiLU evaluated only at the events
    (by the fused extraction, from the conv input x), the gather and the
    depthwise flat scan as one autograd node: no dense x_conv is written or
    read, forward or backward. The backward runs the scan backward to du and
    then bcm_causal_conv1d_bwd_events, which writes dx (x's strides),
    dweight and dbias from du. Same values as the dense conv followed by
    _IndexedScanFn (dweight / dbias up to summation order)."""

    @staticmethod
    def forward(ctx, x, weight, bias, payload, event_index, k_flat, cu_seqlens, max_seqlen: int, dt_idle, dt_active,
                A, W_B, W_C, D):
        ctx.event_index, ctx.has_bias = event_index, bias is not None
        out, saved = _event_scan_fwd(ctx, payload[0], k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, W_B,
                                     W_C, D)
        ctx.n_scan = len(saved)
        ctx.save_for_backward(*saved, x, weight, *([bias] if bias is not None else []))
        return out

    @staticmethod
    def backward(ctx, dout):
        saved = ctx.saved_tensors
        x, weight = saved[ctx.n_scan], saved[ctx.n_scan + 1]
        bias = saved[ctx.n_scan + 2] if ctx.has_bias else None
        with cuda_stage("sparse_scan_backward"):
            du, *grads = _event_scan_bwd(ctx, saved[:ctx.n_scan], dout)
        with cuda_stage("conv_backward"):
            dx, dw, db = conv1d_bwd_events(x, weight, bias, True, du, ctx.event_index)
        return (dx, dw.to(weight.dtype), db.to(bias.dtype) if db is not None else None, None, None, None, None, None,
                *grads)


class _IndexedRestoreFn(torch.autograd.Function):
    """Zero-order-hold restore reading the event index of the fused
    extraction (same result as RestoreDenseFn)."""

    @staticmethod
    def forward(ctx, y_flat, event_index, n_ch: int, dim: int, seqlen: int):
        ctx.event_index, ctx.n_ch, ctx.dim, ctx.seqlen = event_index, n_ch, dim, seqlen
        ctx.n_events = int(y_flat.size(0))
        return restore_dense_cuda_nodecay.restore_fwd_indexed(y_flat, event_index, n_ch, dim, seqlen)

    @staticmethod
    def backward(ctx, dout):
        dout = dout.contiguous()
        dy = torch.empty(ctx.n_events, dtype=torch.float32, device=dout.device)
        with cuda_stage("restore_backward"):
            restore_dense_cuda_nodecay.restore_bwd_indexed(dout, ctx.event_index, ctx.n_ch, ctx.dim, ctx.seqlen, dy)
        return dy, None, None, None, None


class _IndexedRestoreProjFn(torch.autograd.Function):
    """The restore followed by out_proj in one op, reading the event index of
    the fused extraction. The dense restore output z [B, L, d_inner] is not
    kept for the backward and its gradient dz is never formed: dy comes from
    one kernel that computes dz tile by tile on the matrix cores and runs
    the restore backward's sweep on it (bcm_restore_proj_bwd).

    mode "gemm": z is formed for the forward GEMM (and again for the weight
    gradient's split-K GEMM) and freed, hipBLASLt runs the two products.
    mode "mfma": the forward and the weight gradient also run as this
    package's kernels, with z generated from the event index inside them
    (bcm_restore_proj_fwd, bcm_restore_proj_bwd): no dense z at all.
    Same result as projections.linear(_IndexedRestoreFn.apply(...), weight,
    bias), in another fp32 summation order."""

    @staticmethod
    def forward(ctx, y_flat, weight, bias, event_index, n_ch: int, dim: int, seqlen: int, mode: str):
        ctx.event_index, ctx.n_ch, ctx.dim, ctx.seqlen, ctx.mode = event_index, n_ch, dim, seqlen, mode
        ctx.has_bias = bias is not None
        ctx.save_for_backward(y_flat, weight)
        if mode == "mfma":
            return restore_dense_cuda_nodecay.restore_proj_fwd_indexed(y_flat, event_index, n_ch, dim, seqlen,
                                                                        weight, bias)
        z = restore_dense_cuda_nodecay.restore_fwd_indexed(y_flat, event_index, n_ch, dim, seqlen)
        return F.linear(z, weight, bias)

    @staticmethod
    def backward(ctx, dout):
        y_flat, weight = ctx.saved_tensors
        mfma = ctx.mode == "mfma"
        need_dy, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dout = dout.contiguous()
        with cuda_stage("restore_backward"):
            dy, dw = restore_dense_cuda_nodecay.restore_proj_bwd_indexed(
                dout, y_flat, ctx.event_index, ctx.n_ch, ctx.dim, ctx.seqlen, weight, need_dy=need_dy,
                need_dw=need_dw and mfma)
        if need_dw and not mfma:
            z = restore_dense_cuda_nodecay.restore_fwd_indexed(y_flat, ctx.event_index, ctx.n_ch, ctx.dim, ctx.seqlen)
            dw = projections.weight_grad(dout.reshape(-1, dout.size(-1)), z.reshape(-1, ctx.dim))
        db = dout.sum((0, 1)) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return dy, dw, db, None, None, None, None, None


class TwoLevelDelta(nn.Module):
    """Per-channel idle / active steps: dt = softplus(a) + eps (e_model.py:210-230)."""

    def __init__(self, d_inner: int, dt_min=0.001, dt_max=0.1, dt_init_floor=1e-4, eps=1e-6, device=None):
        super().__init__()
        self.eps = eps
        scale = math.log(dt_max) - math.log(dt_min)
        rand0 = torch.rand(d_inner, device=device) * scale + math.log(dt_min)
        rand1 = torch.rand(d_inner, device=device) * scale + math.log(dt_min)
        dt0 = torch.exp(rand0).clamp(min=dt_init_floor)
        dt1 = torch.exp(rand1).clamp(min=dt_init_floor)

        def inv_sp(y, eps=1e-6):
            y = y.clamp_min(eps)
            return torch.log(torch.expm1(y))

        self.a0 = nn.Parameter(inv_sp(dt0))
        self.a1 = nn.Parameter(inv_sp(dt1))

    def levels(self):
        return F.softplus(self.a0) + self.eps, F.softplus(self.a1) + self.eps


class _SpikeBitsFn(torch.autograd.Function):
    """The "ste" spike s = (p >= thr) + p - p with its identity gradient, as
    one kernel that also emits the event bitmask of the transposed spikes
    (bcm_spike_bits). The bitmask rides on s as `_bcm_event_bits` =
    (bitmask, threshold, s._version) for the next block's extraction."""

    @staticmethod
    def forward(ctx, p, threshold: float):
        s, bitmask = _ee_cuda.spike_bits(p, threshold)
        s._bcm_event_bits = (bitmask, threshold, s._version)
        return s

    @staticmethod
    def backward(ctx, grad_s):
        return grad_s, None


def _event_bits_of(s, extract_threshold):
    """The bitmask a spike tensor carries, if it still describes s and the
    extraction's strict s > extract_threshold selects exactly the spikes:
    s is exactly 0 without a spike and within 2^-6 of 1 with one (any
    dtype), so any threshold in [0, 0.9) does."""
    bits = getattr(s, "_bcm_event_bits", None)
    if bits is None or bits[2] != s._version or not (0.0 <= extract_threshold < 0.9):
        return None
    return bits[0]


class SpikeSamplerSurrogate(nn.Module):
    """Bernoulli / threshold spike sampler with a straight-through gradient
    (e_model.py:233-254). With fused_bits (default) the "ste" mode on a
    contiguous [B, L, D] CUDA tensor runs as one kernel that also emits the
    event bitmask the next block's extraction reads (bcm_spike_bits): same
    values and gradient."""

    def __init__(self, mode: str = "ste", sample_inference: bool = False, threshold: float = 0.5,
                 fused_bits: bool = True):
        super().__init__()
        assert mode in ("prob", "ste")
        self.mode, self.sample_inference, self.threshold = mode, sample_inference, threshold
        self.fused_bits = fused_bits

    def forward(self, p):
        if (self.mode == "ste" and self.fused_bits and p.is_cuda and p.dim() == 3 and p.is_contiguous()
                and p.dtype in (torch.float32, torch.float16, torch.bfloat16)):
            return _SpikeBitsFn.apply(p, float(self.threshold))
        if self.mode == "prob":
            if self.training:
                s = torch.bernoulli(p)
                return s.detach() + p - p.detach()
            if self.sample_inference:
                return torch.bernoulli(p)
            return (p >= self.threshold).to(dtype=p.dtype)
        s = (p >= self.threshold).to(dtype=p.dtype)
        return s.detach() + p - p.detach()


class Mamba(nn.Module):
    """Event-driven Mamba block (e_model.py:258-506), same parameters and
    initialisation as the reference."""

    def __init__(self, d_model, d_state=16, d_conv=4, expand=2, dt_rank="auto", dt_min=0.001, dt_max=0.1,
                 dt_init="random", dt_scale=1.0, dt_init_floor=1e-4, conv_bias=True, bias=False,
                 use_fast_path=False, spiking=True, spike_mode="ste", prob_activation="sigmoid",
                 sample_inference=False, threshold=0.5, layer_idx=None, device=None, dtype=None,
                 fused_event_path=True, conv_at_events=True, fused_out_proj=True):
        factory_kwargs = {"device": device, "dtype": dtype}
        super().__init__()
        self.d_model, self.d_state, self.d_conv, self.expand = d_model, d_state, d_conv, expand
        self.d_inner = int(self.expand * self.d_model)
        self.dt_rank = math.ceil(self.d_model / 16) if dt_rank == "auto" else dt_rank
        self.use_fast_path = use_fast_path
        self.layer_idx = layer_idx
        self.spiking = spiking
        assert spike_mode in ("ste", "prob")
        assert prob_activation in ("sigmoid", "clamp")
        self.spike_mode, self.prob_activation = spike_mode, prob_activation
        self.sample_inference, self.threshold = sample_inference, threshold
        self.scan_impl = "flat_ch"
        self.fused_event_path = fused_event_path
        self.conv_at_events = conv_at_events
        self.fused_out_proj = fused_out_proj

        self.in_proj = nn.Linear(self.d_model, self.d_inner, bias=bias, **factory_kwargs)
        self.conv1d = nn.Conv1d(in_channels=self.d_inner, out_channels=self.d_inner, bias=conv_bias,
                                kernel_size=d_conv, groups=self.d_inner, padding=d_conv - 1, **factory_kwargs)
        self.activation = "silu"
        self.act = nn.SiLU()
        fp32_kwargs = {"device": device, "dtype": torch.float32}
        self.W_BC = nn.Parameter(torch.empty(self.d_inner, self.d_state * 2, **fp32_kwargs))
        nn.init.normal_(self.W_BC, std=0.02)
        self.D = nn.Parameter(torch.ones(self.d_inner, **fp32_kwargs))
        self.D._no_weight_decay = True
        A = repeat(torch.arange(1, self.d_state + 1, dtype=torch.float32, device=device), "n -> d n",
                   d=self.d_inner).contiguous()
        self.A_log = nn.Parameter(torch.log(A))
        self.A_log._no_weight_decay = True
        self.out_proj = nn.Linear(self.d_inner, self.d_model, bias=bias, **factory_kwargs)
        self.prob_head = nn.Linear(self.d_model, self.d_model, bias=True, **factory_kwargs)
        self.spike_sampler = SpikeSamplerSurrogate(mode=self.spike_mode, sample_inference=self.sample_inference,
                                                   threshold=self.threshold)
        self.delta_gen = TwoLevelDelta(self.d_inner, dt_min=dt_min, dt_max=dt_max, dt_init_floor=dt_init_floor,
                                       device=device)

    def to_spike(self, out):
        logits = projections.linear(out, self.prob_head.weight, self.prob_head.bias) if self.fused_event_path \
            else self.prob_head(out)
        p = torch.sigmoid(logits) if self.prob_activation == "sigmoid" else torch.clamp(logits, 0.0, 1.0)
        return self.spike_sampler(p)

    def _to_spike(self, out):
        return self.to_spike(out) if self.spiking else out

    def extract_events_1d(self, hidden_states, x_conv, threshold: float):
        """Reference composition (e_model.py:361-409): base extraction,
        expansion, host read of max_seqlen, differentiable gather."""
        B, L, d_model = hidden_states.shape
        assert d_model == self.d_model, f"hidden_states last dim {d_model} != self.d_model {self.d_model}"
        base_input = rearrange(hidden_states, "b l d -> b d l").contiguous()
        with cuda_stage("routing_index_extraction"):
            base_ch_ids, base_t_steps, base_k_flat, base_cu_seqlens, _counts, _ms = \
                _ee_cuda.extract_base_events(base_input, threshold)
        with cuda_stage("active_token_packing"):
            channel_ids, time_steps, k_flat, cu_seqlens, max_seqlen_t = _ee_cuda.expand_base_events(
                base_ch_ids, base_t_steps, base_k_flat, base_cu_seqlens, B, self.d_model, self.expand)
            max_seqlen = int(max_seqlen_t.item())
        with cuda_stage("active_gather_forward"):
            x_conv_flat = _gather_events_fn(x_conv, channel_ids, time_steps)
        return channel_ids, time_steps, k_flat, cu_seqlens, max_seqlen, x_conv_flat

    def _conv(self, x, seqlen):
        """silu(conv1d(x)[..., :L]) (e_model.py:442-451). The fused path runs
        it as the HIP causal conv (causal_conv1d_fn, the reference's fast
        path); the reference composition keeps nn.Conv1d, its fallback."""
        if self.fused_event_path:
            return causal_conv1d_fn(x, self.conv1d.weight[:, 0, :], self.conv1d.bias, activation="silu")
        return self.act(self.conv1d(x)[..., :seqlen])

    def _conv_at_events_ok(self, x):
        """The fused path evaluates the conv at the events when x's rows are
        contiguous and 4-step aligned (bcm_causal_conv1d_bwd_events)."""
        es = x.element_size()
        (s_in, n_in), (s_out, _) = sorted(((x.stride(1), x.size(1)), (x.stride(0), x.size(0))))
        rows_apart = s_in >= x.size(2) and s_out >= s_in * n_in  # dx reuses x's strides
        return (self.fused_event_path and self.conv_at_events and x.stride(2) == 1 and x.size(2) % 4 == 0
                and x.stride(0) % 4 == 0 and x.stride(1) % 4 == 0 and x.data_ptr() % (4 * es) == 0 and rows_apart
                and self.d_conv <= 8 and x.dtype in (torch.float32, torch.float16, torch.bfloat16))

    def _restore_proj_ok(self, y_flat, seqlen):
        """The restore -> out_proj op applies (fp32, 32-bit offsets; in the
        all-kernel mode, d_inner within the forward kernel's LDS: 16 bytes of
        index words per channel beside 36 KB of operand buffers on a 160 KB
        part, so up to 7936 channels)."""
        w, b = self.out_proj.weight, self.out_proj.bias
        f32 = torch.float32
        return (self.fused_out_proj and y_flat.dtype == f32 and w.dtype == f32 and w.is_contiguous()
                and (b is None or b.dtype == f32) and y_flat.numel() * 4 < 2 ** 31
                and seqlen * self.d_model * 4 < 2 ** 31 and self.d_model * self.d_inner * 4 < 2 ** 31
                and (self.fused_out_proj != "mfma" or self.d_inner <= 7936))

    def forward(self, hidden_states, inference_params=None):
        if inference_params is not None:
            raise RuntimeError("Mamba: the decode / inference-cache path is not part of the event-path build")
        batch, seqlen, dim = hidden_states.shape
        if self.fused_event_path:  # the same product, with the split-K weight gradient
            xw = projections.proj_tokens_last(self.in_proj.weight, hidden_states.reshape(batch * seqlen, dim))
        else:
            xw = self.in_proj.weight @ rearrange(hidden_states, "b l d -> d (b l)")
        x = rearrange(xw, "d (b l) -> b d l", l=seqlen)
        if self.in_proj.bias is not None:
            x = x + rearrange(self.in_proj.bias.to(dtype=x.dtype), "d -> d 1")
        conv_ev = self._conv_at_events_ok(x)
        if not conv_ev:
            x = self._conv(x, seqlen).contiguous()

        dt_idle, dt_active = self.delta_gen.levels()
        A = -torch.exp(self.A_log)
        W_B = self.W_BC[:, :self.d_state].contiguous()
        W_C = self.W_BC[:, self.d_state:].contiguous()
        n_ch = batch * self.d_inner

        if self.fused_event_path:
            # spikes from a fused STE head carry their event bitmask: no
            # transposed copy of the membrane and no count pass over it
            bits = _event_bits_of(hidden_states, self.threshold)
            base_input = None if bits is not None else \
                rearrange(hidden_states.detach(), "b l d -> b d l").contiguous()
            w_conv, b_conv = self.conv1d.weight[:, 0, :], self.conv1d.bias
            with cuda_stage("routing_index_extraction"):
                _ch, time_steps, k_flat, cu_seqlens, max_seqlen, x_ev, event_index = \
                    _ee_cuda.extract_events_indexed(base_input, self.threshold, self.expand, x.detach(),
                                                    positions=False, conv=(w_conv, b_conv, True) if conv_ev else None,
                                                    bits=(bits, (batch, dim, seqlen)) if bits is not None else None)
            with cuda_stage("sparse_scan_forward"):
                if conv_ev:  # x is the conv input: silu(conv(x)) exists only at the events
                    y_flat = _IndexedConvScanFn.apply(x, w_conv, b_conv, (x_ev,), event_index, k_flat, cu_seqlens,
                                                      int(max_seqlen), dt_idle, dt_active, A, W_B, W_C, self.D)
                else:
                    y_flat = _IndexedScanFn.apply(x, (x_ev,), event_index, k_flat, cu_seqlens, int(max_seqlen),
                                                  dt_idle, dt_active, A, W_B, W_C, self.D)
        else:
            _ch, time_steps, k_flat, cu_seqlens, max_seqlen, x_conv_flat = self.extract_events_1d(
                hidden_states, x, self.threshold)
            with cuda_stage("sparse_scan_forward"):
                y_flat, _ = selective_scan_flat_ch_fn(x_conv_flat, k_flat, cu_seqlens, int(max_seqlen), dt_idle,
                                                      dt_active, A, W_B, W_C, self.D, None, tile_offsets=None,
                                                      tile_chunk_size=0, is_depthwise_bc=True, pw_B=None,
                                                      pw_C=None)
        with cuda_stage("dense_restoration_forward"):
            if self.fused_event_path and self._restore_proj_ok(y_flat, seqlen):
                return _IndexedRestoreProjFn.apply(y_flat, self.out_proj.weight, self.out_proj.bias, event_index,
                                                   n_ch, self.d_inner, seqlen,
                                                   "mfma" if self.fused_out_proj == "mfma" else "gemm")
            if self.fused_event_path:
                y_dense = _IndexedRestoreFn.apply(y_flat, event_index, n_ch, self.d_inner, seqlen)
            else:
                y_dense = restore_dense_fn(y_flat, time_steps.to(torch.int32), cu_seqlens, self.d_inner, seqlen)
        if self.fused_event_path:
            return projections.linear(y_dense, self.out_proj.weight, self.out_proj.bias)
        return self.out_proj(y_dense)
