"""Drop-in for the reference extension module `restore_dense_cuda_nodecay`
(csrc/r_nodecay/restore_dense.cpp, bindings :207-226), backed by the HIP
restore kernels of libbcm_event_scan.so.

restore_dense_fwd(y_flat, time_steps, cu_seqlens, dim, seqlen, out_dtype=None)
    -> (B, L, D): out[b, t, d] = y of the last event of channel b*dim+d at or
       before t (zero-order hold), 0 before the channel's first event.
restore_dense_bwd(dout, time_steps, cu_seqlens, dim, seqlen)
    -> dy (E,) float32: sum of dout over the steps each event holds.

time_steps must be strictly increasing inside each channel (as produced by
extraction). Unlike the reference (exact up to 4095 events per channel),
every channel length is exact.
"""
import torch

try:
    from . import _native as _nat
    from . import _provenance as _prov
except ImportError:  # imported with this directory on sys.path
    import _native as _nat
    import _provenance as _prov

__all__ = ["restore_dense_fwd", "restore_dense_bwd", "build_event_index", "restore_fwd_indexed",
           "restore_bwd_indexed", "restore_proj_fwd_indexed", "restore_proj_bwd_indexed"]

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def build_event_index(time_steps, cu_seqlens, seqlen, zero_f32=None):
    """(bitmask, tile_start) of per-channel sorted time steps; optionally
    zero-fills the float32 tensor zero_f32 in the same launch."""
    n_ch = int(cu_seqlens.size(0)) - 1
    dev = time_steps.device
    bitmask = torch.empty((n_ch, _nat.bitmask_words(seqlen)), dtype=torch.int32, device=dev)
    tile_start = torch.empty((n_ch, _nat.tile_count(seqlen) + 1), dtype=torch.int32, device=dev)
    _nat.call("bcm_build_event_index", _nat.ptr(time_steps), _nat.ptr(cu_seqlens), n_ch, int(seqlen),
              _nat.ptr(bitmask), _nat.ptr(tile_start), _nat.ptr(zero_f32),
              int(zero_f32.numel()) if zero_f32 is not None else 0, _nat.stream_of(time_steps))
    return bitmask, tile_start


def restore_fwd_indexed(y_flat, event_index, n_ch, dim, seqlen, out_dtype=None):
    """Restore forward from an event index (bitmask, tile_start, expand)."""
    bitmask, tile_start, mrd = event_index
    out_dtype = y_flat.dtype if out_dtype is None else out_dtype
    out = torch.empty((n_ch // dim, seqlen, dim), dtype=out_dtype, device=y_flat.device)
    _nat.call("bcm_restore_fwd", _nat.ptr(y_flat), _nat.dtype_code(y_flat.dtype), int(y_flat.numel()),
              _nat.ptr(bitmask), int(mrd),
              _nat.ptr(tile_start), n_ch, int(dim), int(seqlen), _nat.ptr(out), _nat.dtype_code(out_dtype),
              _nat.stream_of(y_flat))
    return out


_sync_areas = {}  # (device index, stream handle) -> int64 tensor, zero between calls
_cu_counts = {}  # device index -> compute units


def _chained_fits(n_ch, dim, seqlen, dev):
    """The one-kernel restore backward where its tile grid fits one launch
    (at most 16 waves per compute unit), else the two-pass form: the
    one-kernel form's later launches cannot overlap the earlier ones."""
    key = dev.index
    if key not in _cu_counts:
        _cu_counts[key] = torch.cuda.get_device_properties(dev).multi_processor_count
    waves = (n_ch // dim) * _nat.tile_count(seqlen) * -(-dim // 64)
    return waves <= 16 * _cu_counts[key]


def _sync_area(dev, n_ch, seqlen):
    """The stream's sync area for bcm_restore_bwd_chained, zeroed once when
    it is made (or grown); every completed call leaves it zero. One area per
    stream: the calls that share it are ordered by that stream."""
    nbytes = int(_nat.lib().bcm_restore_bwd_sync_bytes(n_ch, seqlen))
    key = (dev.index, _nat.stream_of_device(dev).value)
    area = _sync_areas.get(key)
    if area is None or 8 * area.numel() < nbytes:
        area = _sync_areas[key] = torch.zeros(nbytes // 8, dtype=torch.int64, device=dev)
    return area


def restore_bwd_indexed(dout, event_index, n_ch, dim, seqlen, dy, chained=None):
    """Restore backward from an event index into the float32 dy (every
    event's entry is written; no zero-init needed). chained: True for the
    one-kernel form (bcm_restore_bwd_chained, whose look-back relies on the
    index being the extraction's own), False for the two-pass form
    (bcm_restore_bwd), None to choose by size (the one-kernel form where it
    fits one launch)."""
    bitmask, tile_start, mrd = event_index
    dev = dout.device
    if chained is None:
        chained = _chained_fits(n_ch, dim, seqlen, dev)
    if chained:
        area = _sync_area(dev, n_ch, seqlen)
        _nat.call("bcm_restore_bwd_chained", _nat.ptr(dout), _nat.dtype_code(dout.dtype), _nat.ptr(bitmask),
                  int(mrd), _nat.ptr(tile_start), n_ch, int(dim), int(seqlen), _nat.ptr(dy), _nat.F32,
                  int(dy.numel()), _nat.ptr(area), 8 * area.numel(), _nat.stream_of(dout))
        return dy
    ws = torch.empty(_nat.lib().bcm_restore_bwd_workspace_bytes(n_ch, seqlen) // 4, dtype=torch.float32,
                     device=dev)
    _nat.call("bcm_restore_bwd", _nat.ptr(dout), _nat.dtype_code(dout.dtype), _nat.ptr(bitmask), int(mrd),
              _nat.ptr(tile_start), n_ch, int(dim), int(seqlen), _nat.ptr(dy), int(dy.numel()), _nat.ptr(ws),
              4 * ws.numel(),
              _nat.stream_of(dout))
    return dy


def restore_proj_fwd_indexed(y_flat, event_index, n_ch, dim, seqlen, weight, bias=None):
    """The restore followed by the block's out_proj, without the dense
    restore output (bcm_restore_proj_fwd): F.linear(restore(y_flat), weight,
    bias) as (B, L, d_model) float32. fp32 y_flat, weight and bias."""
    fn = "restore_proj_fwd_indexed"
    _check(y_flat.dtype == torch.float32 and weight.dtype == torch.float32, f"{fn}: fp32 y_flat and weight")
    _check(bias is None or bias.dtype == torch.float32, f"{fn}: fp32 bias")
    _check(weight.dim() == 2 and weight.size(1) == dim and weight.is_contiguous(), f"{fn}: weight [d_model, dim]")
    bitmask, tile_start, mrd = event_index
    dm = weight.size(0)
    out = torch.empty((n_ch // dim, seqlen, dm), dtype=torch.float32, device=y_flat.device)
    _nat.call("bcm_restore_proj_fwd", _nat.ptr(y_flat), int(y_flat.numel()), _nat.ptr(bitmask), int(mrd),
              _nat.ptr(tile_start), n_ch, int(dim), int(seqlen), _nat.ptr(weight),
              _nat.ptr(bias.contiguous()) if bias is not None else None, dm, _nat.ptr(out), _nat.stream_of(y_flat))
    return out


def restore_proj_bwd_indexed(dout, y_flat, event_index, n_ch, dim, seqlen, weight, need_dy=True, need_dw=True):
    """Backward of restore_proj_fwd_indexed (bcm_restore_proj_bwd) from dout
    (B, L, d_model): (dy float32 [E] or None, dweight [d_model, dim] or
    None). The bias gradient is dout's column sum (not computed here)."""
    bitmask, tile_start, mrd = event_index
    dout = dout.contiguous()
    dm = weight.size(0)
    # the weight gradient's partials (d_model x dim per sequence segment) only
    # when it is asked for; dy alone needs the fix-up arrays
    nbytes = _nat.lib().bcm_restore_proj_bwd_workspace_bytes(n_ch, int(dim), int(seqlen), dm) if need_dw else \
        _nat.lib().bcm_restore_bwd_workspace_bytes(n_ch, int(seqlen))
    ws = torch.empty(max(4, nbytes) // 4, dtype=torch.float32, device=dout.device)
    dy = torch.empty(y_flat.numel(), dtype=torch.float32, device=dout.device) if need_dy else None
    dw = torch.empty_like(weight) if need_dw else None
    _nat.call("bcm_restore_proj_bwd", _nat.ptr(dout), _nat.ptr(y_flat), int(y_flat.numel()), _nat.ptr(bitmask),
              int(mrd), _nat.ptr(tile_start), n_ch, int(dim), int(seqlen), _nat.ptr(weight), dm, _nat.ptr(dy),
              _nat.ptr(dw), _nat.ptr(ws), 4 * ws.numel(), _nat.stream_of(dout))
    return dy, dw


def restore_dense_fwd(y_flat, time_steps, cu_seqlens, dim, seqlen, out_dtype=None):
    """Zero-order-hold restore forward (restore_dense.cpp:43-130)."""
    fn = "restore_dense_fwd"
    _check(y_flat.dtype in _FLOATS, f"{fn}: y_flat must be fp32, fp16, or bf16")
    _check(time_steps.dtype == torch.int32, f"{fn}: time_steps must be int32 (torch.int32)")
    _check(cu_seqlens.dtype == torch.int32, f"{fn}: cu_seqlens must be int32 (torch.int32)")
    _check(y_flat.is_cuda and time_steps.is_cuda and cu_seqlens.is_cuda, f"{fn}: all tensors must be on CUDA")
    _check(y_flat.is_contiguous() and time_steps.is_contiguous() and cu_seqlens.is_contiguous(),
           f"{fn}: all tensors must be contiguous")
    _check(y_flat.dim() == 1, f"{fn}: y_flat must be 1-D")
    _check(time_steps.shape == y_flat.shape, f"{fn}: time_steps shape must equal y_flat shape")
    _check(cu_seqlens.dim() == 1, f"{fn}: cu_seqlens must be 1-D")
    dim, seqlen = int(dim), int(seqlen)
    _check(dim >= 1, f"{fn}: dim must be >= 1")
    _check(seqlen >= 1, f"{fn}: seqlen must be >= 1")
    n_ch = int(cu_seqlens.size(0)) - 1
    _check(n_ch >= 1, f"{fn}: cu_seqlens must have at least 2 elements")
    _check(n_ch % dim == 0, f"{fn}: n_channels (B*D) must be divisible by dim")
    out_dtype = y_flat.dtype if out_dtype is None else out_dtype
    _check(out_dtype in _FLOATS, f"{fn}: out_dtype must be fp32, fp16, or bf16")
    if y_flat.dtype == torch.float16:
        _check(out_dtype == torch.float16, f"{fn}: fp16 input only supports fp16 output")
    if y_flat.dtype == torch.bfloat16:
        _check(out_dtype == torch.bfloat16, f"{fn}: bf16 input only supports bf16 output")
    if y_flat.numel() == 0:  # no events: every position precedes its channel's first event
        return torch.zeros((n_ch // dim, seqlen, dim), dtype=out_dtype, device=y_flat.device)
    with torch.cuda.device(y_flat.device):
        idx = _prov.event_index_for(time_steps, cu_seqlens, seqlen)  # the extraction's own, when unchanged
        bitmask, tile_start = idx if idx is not None else build_event_index(time_steps, cu_seqlens, seqlen)
        return restore_fwd_indexed(y_flat, (bitmask, tile_start, 1), n_ch, dim, seqlen, out_dtype)


def restore_dense_bwd(dout, time_steps, cu_seqlens, dim, seqlen):
    """Zero-order-hold restore backward -> dy (E,) float32
    (restore_dense.cpp:138-202)."""
    fn = "restore_dense_bwd"
    _check(dout.dtype in _FLOATS, f"{fn}: dout must be fp32/fp16/bf16")
    _check(time_steps.dtype == torch.int32, f"{fn}: time_steps must be int32")
    _check(cu_seqlens.dtype == torch.int32, f"{fn}: cu_seqlens must be int32")
    _check(dout.is_cuda and time_steps.is_cuda and cu_seqlens.is_cuda, f"{fn}: all tensors must be on CUDA")
    _check(dout.is_contiguous() and time_steps.is_contiguous() and cu_seqlens.is_contiguous(),
           f"{fn}: all tensors must be contiguous")
    dim, seqlen = int(dim), int(seqlen)
    _check(dim >= 1, f"{fn}: dim must be >= 1")
    _check(seqlen >= 1, f"{fn}: seqlen must be >= 1")
    n_ch = int(cu_seqlens.size(0)) - 1
    _check(dout.dim() == 3, f"{fn}: dout must be 3-D (B, L, D)")
    _check(dout.size(1) == seqlen, f"{fn}: dout.size(1) must equal seqlen")
    _check(dout.size(2) == dim, f"{fn}: dout.size(2) must equal dim (D)")
    _check(dout.size(0) * dim == n_ch, f"{fn}: dout.size(0)*dim must equal n_channels")
    dy = torch.empty(int(time_steps.size(0)), dtype=torch.float32, device=dout.device)
    if dy.numel() == 0:
        return dy
    with torch.cuda.device(dout.device):
        idx = _prov.event_index_for(time_steps, cu_seqlens, seqlen)
        if idx is not None:  # the extraction's index: every event is in it, no zero-fill
            restore_bwd_indexed(dout, idx + (1,), n_ch, dim, seqlen, dy)
        else:
            bitmask, tile_start = build_event_index(time_steps, cu_seqlens, seqlen, zero_f32=dy)
            if n_ch > 0:
                restore_bwd_indexed(dout, (bitmask, tile_start, 1), n_ch, dim, seqlen, dy, chained=False)
    return dy
