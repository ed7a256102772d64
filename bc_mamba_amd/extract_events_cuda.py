"""Drop-in for the reference extension module `extract_events_cuda`
(csrc/extract/extract_events_cuda.cu, bindings :759-798), backed by the HIP
kernels of libbcm_event_scan.so.

Same function names, argument order, return lists, dtypes and error style
as the reference; every check raises RuntimeError with the reference's
message. Outputs are allocated with torch on the input's device and filled
by the native library on the current stream.
"""
import torch

import threading

try:
    from . import _native as _nat
    from . import _provenance as _prov
except ImportError:  # imported with this directory on sys.path
    import _native as _nat
    import _provenance as _prov

__all__ = ["extract_events", "extract_base_events", "expand_base_events",
           "gather_events_fwd", "gather_events_bwd", "extract_events_indexed"]

_I32 = torch.int32


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _empty_i32(n, dev):
    return torch.empty(n, dtype=_I32, device=dev)


_metas = threading.local()


def _host_meta(dev):
    """This thread's pinned (E, max_seqlen) words for device dev. Every user
    reads its values before returning, so one pair per thread and device
    serves every call."""
    d = getattr(_metas, "by_dev", None)
    if d is None:
        d = _metas.by_dev = {}
    key = torch.device(dev).index
    if key not in d:
        d[key] = _nat.HostMeta()
    return d[key]


def _count_scan(x2d, dtype_code, threshold):
    """Passes 1-2: bitmask, counts, cu_seqlens, and meta = (E, max) in pinned
    host memory that the offsets kernel writes directly; meta.wait() polls
    it (no copy kernel, no stream sync)."""
    NC, L = x2d.shape
    dev = x2d.device
    bitmask = torch.empty((NC, _nat.bitmask_words(L)), dtype=_I32, device=dev)
    counts = _empty_i32(NC, dev)
    cu = _empty_i32(NC + 1, dev)
    meta = _host_meta(dev)
    meta.arm()
    s = _nat.stream_of(x2d)
    _nat.call("bcm_extract_count", _nat.ptr(x2d), dtype_code, NC, L, float(threshold),
              _nat.ptr(bitmask), _nat.ptr(counts), s)
    _nat.call("bcm_extract_scan", _nat.ptr(counts), NC, _nat.ptr(cu), meta.ptr(), s)
    return bitmask, counts, cu, meta


def extract_base_events(base_input, threshold):
    """base_input [B, d_model, L] fp32/fp16/bf16 -> [ch_ids, t_steps, k_flat,
    cu_seqlens, counts, max_seqlen] (extract_events_cuda.cu:324-418).

    An event is float(base_input[b, d, t]) > float(threshold); events are
    channel-major (channel = b*d_model + d), time-ascending; k = t+1 for a
    channel's first event, else the gap to the previous one. The host reads
    the total event count to size the outputs, like the reference (here by
    polling pinned memory the offsets kernel writes, not by a stream sync).

    The fill also writes the event index (bitmask and tile table), which is
    kept on t_steps, and the host-read longest channel is kept on
    cu_seqlens: restore_dense_fwd / _bwd, gather_events_bwd and the scan
    read them instead of recomputing them while those tensors are unchanged
    (bc_mamba_amd._provenance)."""
    _check(base_input.is_cuda, "base_input must be CUDA")
    _check(base_input.is_contiguous(), "base_input must be contiguous")
    _check(base_input.dim() == 3, "base_input must be 3-D [B, d_model, L]")
    _check(base_input.dtype in (torch.float32, torch.float16, torch.bfloat16),
           "base_input must be fp32, fp16 or bf16")
    B, Dm, L = base_input.shape
    dev = base_input.device
    with torch.cuda.device(dev):
        x2d = base_input.view(B * Dm, L)
        bitmask, counts, cu, meta = _count_scan(x2d, _nat.dtype_code(base_input.dtype), threshold)
        E, max_seqlen = meta.wait(dev)
        _prov.attach_max_seqlen(cu, max_seqlen)
        if E == 0:
            ei = torch.zeros(0, dtype=_I32, device=dev)
            return [ei, ei, ei, cu, counts, torch.zeros(1, dtype=_I32, device=dev)]
        ch, t, k = _empty_i32(E, dev), _empty_i32(E, dev), _empty_i32(E, dev)
        tile_start = torch.empty((B * Dm, _nat.tile_count(L) + 1), dtype=_I32, device=dev)
        _nat.call("bcm_extract_fill", _nat.ptr(bitmask), _nat.ptr(cu), B * Dm, L, 1, None, 0,
                  _nat.ptr(ch), _nat.ptr(t), _nat.ptr(k), None, _nat.ptr(tile_start), None, _nat.stream_of(x2d))
        _prov.attach_event_index(t, ch, cu, L, bitmask, tile_start)
        return [ch, t, k, cu, counts, torch.full((), max_seqlen, dtype=_I32, device=dev)]


def expand_base_events(base_ch_ids, base_t_steps, base_k_flat, base_cu_seqlens, B, d_model, expand):
    """Replicate base channel c into logical channels c*expand + r
    (repeat_interleave order) -> [channel_ids, time_steps, k_flat,
    cu_seqlens, max_seqlen] (extract_events_cuda.cu:529-603)."""
    _check(base_ch_ids.is_cuda, "base_ch_ids must be CUDA")
    _check(base_ch_ids.is_contiguous(), "base_ch_ids must be contiguous")
    NC_base = int(B) * int(d_model)
    NC_inner = NC_base * int(expand)
    E_base = int(base_ch_ids.size(0))
    dev = base_ch_ids.device
    with torch.cuda.device(dev):
        if E_base == 0:
            ei = torch.zeros(0, dtype=_I32, device=dev)
            return [ei, ei, ei, torch.zeros(NC_inner + 1, dtype=_I32, device=dev),
                    torch.zeros(1, dtype=_I32, device=dev)]
        for name, tns in (("base_t_steps", base_t_steps), ("base_k_flat", base_k_flat),
                          ("base_cu_seqlens", base_cu_seqlens)):
            _check(tns.is_cuda and tns.dtype == _I32 and tns.is_contiguous(),
                   f"{name} must be a contiguous int32 CUDA tensor")
        _check(base_ch_ids.dtype == _I32, "base_ch_ids must be int32")
        _check(base_cu_seqlens.numel() >= NC_base + 1, "base_cu_seqlens must have B*d_model+1 entries")
        E = E_base * int(expand)
        ch, t, k = _empty_i32(E, dev), _empty_i32(E, dev), _empty_i32(E, dev)
        cu = _empty_i32(NC_inner + 1, dev)
        s = _nat.stream_of(base_ch_ids)
        _nat.call("bcm_expand_events", _nat.ptr(base_ch_ids), _nat.ptr(base_t_steps), _nat.ptr(base_k_flat),
                  _nat.ptr(base_cu_seqlens), NC_base, E_base, int(expand), _nat.ptr(ch), _nat.ptr(t),
                  _nat.ptr(k), _nat.ptr(cu), s)
        ms = torch.empty((), dtype=_I32, device=dev)
        _nat.call("bcm_seqlen_max", _nat.ptr(base_cu_seqlens), NC_base, _nat.ptr(ms), s)
        base_max = _prov.max_seqlen_of(base_cu_seqlens)
        if base_max is not None:  # every logical channel holds its base channel's events
            _prov.attach_max_seqlen(cu, base_max)
        return [ch, t, k, cu, ms]


def extract_events(mask):
    """LEGACY: bool mask [B, D, L] -> [ch_ids, t_steps, k_flat, cu_seqlens,
    max_seqlen, head_flags] (extract_events_cuda.cu:117-179)."""
    _check(mask.is_cuda, "mask must be a CUDA tensor")
    _check(mask.is_contiguous(), "mask must be contiguous")
    _check(mask.dtype == torch.bool, "mask must be bool")
    B, D, L = mask.shape
    dev = mask.device
    with torch.cuda.device(dev):
        x2d = mask.view(B * D, L)
        bitmask, counts, cu, meta = _count_scan(x2d, _nat.U8, 0.5)
        E, max_seqlen = meta.wait(dev)
        _prov.attach_max_seqlen(cu, max_seqlen)
        if E == 0:
            ei = torch.zeros(0, dtype=_I32, device=dev)
            return [ei, ei, ei, cu, torch.zeros(1, dtype=_I32, device=dev), ei]
        ch, t, k, hf = (_empty_i32(E, dev) for _ in range(4))
        _nat.call("bcm_extract_fill", _nat.ptr(bitmask), _nat.ptr(cu), B * D, L, 1, None, 0,
                  _nat.ptr(ch), _nat.ptr(t), _nat.ptr(k), None, None, _nat.ptr(hf), _nat.stream_of(x2d))
        return [ch, t, k, cu, torch.full((), max_seqlen, dtype=_I32, device=dev), hf]


def gather_events_fwd(x, channel_ids, time_steps):
    """out_x[e] = x.view(NC, L)[channel_ids[e], time_steps[e]] -> [out_x]
    (extract_events_cuda.cu:670-708)."""
    _check(x.is_cuda, "gather_events_fwd: x must be a CUDA tensor")
    _check(x.is_contiguous(), "gather_events_fwd: x must be contiguous")
    _check(channel_ids.dtype == _I32, "gather_events_fwd: channel_ids must be int32")
    _check(time_steps.dtype == _I32, "gather_events_fwd: time_steps must be int32")
    _check(x.dim() == 3, "gather_events_fwd: x must be 3-D [B, D, L]")
    B, D, L = x.shape
    E = int(channel_ids.size(0))
    out = torch.empty(E, dtype=x.dtype, device=x.device)
    if E == 0:
        return [out]
    with torch.cuda.device(x.device):
        _nat.call("bcm_gather_fwd", _nat.ptr(x), _nat.dtype_code(x.dtype), B * D, L,
                  _nat.ptr(channel_ids.contiguous()), _nat.ptr(time_steps.contiguous()), E,
                  _nat.ptr(out), _nat.stream_of(x))
    return [out]


def gather_events_bwd(grad_x, channel_ids, time_steps, NC, L):
    """dx [NC, L] = 0 except dx[channel_ids[e], time_steps[e]] = grad_x[e]
    -> [dx] (extract_events_cuda.cu:717-754). (ch, t) pairs must be unique.
    For the streams of extract_base_events (unchanged), dx is written row
    by row from the extraction's event index (bcm_gather_bwd_rows: no zero
    pass, no scatter; the same values)."""
    _check(grad_x.is_cuda, "gather_events_bwd: grad tensor must be CUDA")
    _check(channel_ids.dtype == _I32, "gather_events_bwd: channel_ids must be int32")
    _check(time_steps.dtype == _I32, "gather_events_bwd: time_steps must be int32")
    NC, L = int(NC), int(L)
    dx = torch.empty((NC, L), dtype=grad_x.dtype, device=grad_x.device)
    with torch.cuda.device(grad_x.device):
        g = grad_x.contiguous()
        idx = _prov.event_index_for(time_steps, None, L, channel_ids)
        if (idx is not None and idx[0].size(0) == NC and g.dim() == 1 and g.size(0) == time_steps.size(0)
                and g.dtype in (torch.float32, torch.float16, torch.bfloat16)):
            _nat.call("bcm_gather_bwd_rows", _nat.ptr(g), _nat.dtype_code(g.dtype), _nat.ptr(idx[0]), 1,
                      _nat.ptr(idx[1]), NC, L, _nat.ptr(dx), _nat.stream_of(g))
            return [dx]
        _nat.call("bcm_gather_bwd", _nat.ptr(g), _nat.dtype_code(g.dtype), _nat.ptr(channel_ids.contiguous()),
                  _nat.ptr(time_steps.contiguous()), int(g.size(0)), NC, L, _nat.ptr(dx), _nat.stream_of(g))
    return [dx]


def _extract_indexed_exact(base_input, threshold, expand, x, positions):
    """extract_events_indexed with the separate offsets pass: E is read
    before the fill, which then writes exactly E events."""
    B, Dm, L = base_input.shape
    dev = base_input.device
    with torch.cuda.device(dev):
        x2d = base_input.view(B * Dm, L)
        bitmask, counts, base_cu, meta = _count_scan(x2d, _nat.dtype_code(base_input.dtype), threshold)
        E_base, max_seqlen = meta.wait(dev)
        NCi = B * Dm * expand
        cu = base_cu if expand == 1 else _empty_i32(NCi + 1, dev)
        s = _nat.stream_of(x2d)
        if expand != 1:
            _nat.call("bcm_expand_events", None, None, None, _nat.ptr(base_cu), B * Dm, 0, expand,
                      None, None, None, _nat.ptr(cu), s)
        E = E_base * expand
        k = _empty_i32(E, dev)
        ch, t = (_empty_i32(E, dev), _empty_i32(E, dev)) if positions else (None, None)
        tile_start = torch.empty((NCi, _nat.tile_count(L) + 1), dtype=_I32, device=dev)
        xe = torch.empty(E, dtype=x.dtype, device=dev) if x is not None else None
        if B * Dm > 0 and L > 0:
            _nat.call("bcm_extract_fill", _nat.ptr(bitmask), _nat.ptr(base_cu), B * Dm, L, expand,
                      _nat.ptr(x), _nat.dtype_code(x.dtype) if x is not None else 0, _nat.ptr(ch), _nat.ptr(t),
                      _nat.ptr(k), _nat.ptr(xe), _nat.ptr(tile_start), None, s)
        return ch, t, k, cu, max_seqlen, xe, (bitmask, tile_start, expand)


def spike_bits(p, threshold, want_s=True):
    """The straight-through spike head (SpikeSamplerSurrogate mode "ste",
    e_model.py:233-254) on p [B, L, Dm] as one kernel (bcm_spike_bits):
    returns (s, bitmask) with s = (p >= threshold) + p - p (None unless
    want_s) and the event bitmask [B*Dm, words] of the transposed spikes,
    ready for extract_events_indexed(bits=...)."""
    _check(p.is_cuda and p.is_contiguous() and p.dim() == 3, "p must be a contiguous 3-D CUDA tensor [B, L, Dm]")
    _check(p.dtype in (torch.float32, torch.float16, torch.bfloat16), "p must be fp32, fp16 or bf16")
    B, L, Dm = p.shape
    bitmask = torch.empty((B * Dm, _nat.bitmask_words(L)), dtype=_I32, device=p.device)
    s = torch.empty_like(p) if want_s else None
    with torch.cuda.device(p.device):
        _nat.call("bcm_spike_bits", _nat.ptr(p), _nat.dtype_code(p.dtype), B, L, Dm, float(threshold),
                  _nat.ptr(bitmask), _nat.ptr(s), _nat.stream_of(p))
    return s, bitmask


def extract_events_indexed(base_input, threshold, expand=1, x=None, positions=True, exact_alloc=False, conv=None,
                           bits=None):
    """Fused extraction for the block forward (no reference counterpart; the
    reference composes extract_base_events + expand_base_events +
    gather_events_fwd). Returns (channel_ids, time_steps, k_flat, cu_seqlens,
    max_seqlen as a Python int, x_events or None, event_index) where
    event_index = (bitmask, tile_start, expand) feeds the restore and the
    row-wise gather backward. With positions=False channel_ids and
    time_steps are None and never written (the indexed restore and gather
    do not use them). One host sync (E and max_seqlen together).

    By default the fill derives the row offsets itself from the count pass's
    block sums (no offsets kernel) and is enqueued before E is known, so its
    event outputs are written into buffers sized for every possible event
    (B*d_model*expand*L); once E is read, the first E entries are copied into
    exact-size tensors and the worst-case buffers are released, so the
    returned streams (which autograd keeps until the backward) hold E
    entries. exact_alloc=True runs the separate offsets pass, reads E first
    and fills exact-size tensors directly (no copies, one more kernel and
    the GPU idle during the host read).

    conv = (weight [D, K], bias [D] or None, silu): x is then the input of
    the block's depthwise causal conv (rows contiguous, any batch / channel
    strides, e.g. the in_proj GEMM output viewed as [B, D, L]) and x_events
    is silu(conv(x)) evaluated at the events only, the values the dense
    conv followed by the gather would give (bcm_extract_fill_blocks_conv).

    bits = (bitmask, (B, d_model, L)): the rows' event bitmask is already
    built (spike_bits, the bits of base_input > threshold); base_input is
    then not read and may be None, and the count pass only counts bits."""
    if bits is not None:
        bits_mask, (B, Dm, L) = bits
        _check(bits_mask.is_cuda and bits_mask.dtype == _I32 and bits_mask.is_contiguous()
               and tuple(bits_mask.shape) == (B * Dm, _nat.bitmask_words(L)), "bits must be [B*d_model, words] int32")
        _check(not exact_alloc and B * Dm > 0 and L > 0, "bits need the fused fill and a non-empty batch")
        dev = bits_mask.device
    else:
        _check(base_input.is_cuda and base_input.is_contiguous() and base_input.dim() == 3,
               "base_input must be a contiguous 3-D CUDA tensor [B, d_model, L]")
        B, Dm, L = base_input.shape
        dev = base_input.device
    expand = int(expand)
    NC = B * Dm
    if conv is not None:
        _check(x is not None and x.is_cuda and x.dim() == 3 and tuple(x.shape) == (B, Dm * expand, L)
               and x.stride(2) == 1, "x must be a CUDA tensor [B, d_model*expand, L] with contiguous rows")
        _check(not exact_alloc, "conv needs the fused fill (exact_alloc=False)")
        if NC == 0 or L == 0:
            r = _extract_indexed_exact(base_input, threshold, expand, None, positions)
            return r[:5] + (torch.empty(0, dtype=x.dtype, device=dev),) + r[6:]
    elif x is not None:
        _check(x.is_cuda and x.is_contiguous() and tuple(x.shape) == (B, Dm * expand, L),
               "x must be a contiguous CUDA tensor [B, d_model*expand, L]")
    if exact_alloc or NC == 0 or L == 0:
        return _extract_indexed_exact(base_input, threshold, expand, x, positions)
    with torch.cuda.device(dev):
        s = _nat.stream_of(bits[0] if bits is not None else base_input)
        NCi, cap = NC * expand, NC * expand * L
        bitmask = bits[0] if bits is not None else torch.empty((NC, _nat.bitmask_words(L)), dtype=_I32, device=dev)
        counts = _empty_i32(NC, dev)
        bsums = _empty_i32(_nat.lib().bcm_extract_block_sums_bytes(NC) // 4, dev)
        cu = _empty_i32(NCi + 1, dev)
        k = _empty_i32(cap, dev)
        ch, t = (_empty_i32(cap, dev), _empty_i32(cap, dev)) if positions else (None, None)
        tile_start = torch.empty((NCi, _nat.tile_count(L) + 1), dtype=_I32, device=dev)
        xe = torch.empty(cap, dtype=x.dtype, device=dev) if x is not None else None
        meta = _host_meta(dev)
        meta.arm()
        if bits is not None:
            _nat.call("bcm_extract_count_bits", _nat.ptr(bitmask), NC, L, _nat.ptr(counts), _nat.ptr(bsums), s)
        else:
            _nat.call("bcm_extract_count_blocks", _nat.ptr(base_input), _nat.dtype_code(base_input.dtype), NC, L,
                      float(threshold), _nat.ptr(bitmask), _nat.ptr(counts), _nat.ptr(bsums), s)
        if conv is None:
            _nat.call("bcm_extract_fill_blocks", _nat.ptr(bitmask), _nat.ptr(counts), _nat.ptr(bsums), meta.ptr(),
                      NC, L, expand, _nat.ptr(x), _nat.dtype_code(x.dtype) if x is not None else 0, _nat.ptr(cu),
                      _nat.ptr(ch), _nat.ptr(t), _nat.ptr(k), _nat.ptr(xe), _nat.ptr(tile_start), s)
        else:
            w, b, silu = conv
            w = w.detach().float().contiguous()
            b = b.detach().float().contiguous() if b is not None else None
            _check(w.dim() == 2 and w.size(0) == Dm * expand and 1 <= w.size(1) <= 8, "conv weight must be [D, K<=8]")
            _nat.call("bcm_extract_fill_blocks_conv", _nat.ptr(bitmask), _nat.ptr(counts), _nat.ptr(bsums),
                      meta.ptr(), NC, L, expand, _nat.ptr(x), _nat.dtype_code(x.dtype), x.stride(0), x.stride(1),
                      Dm * expand, _nat.ptr(w), _nat.ptr(b), int(w.size(1)), int(bool(silu)), _nat.ptr(cu),
                      _nat.ptr(ch), _nat.ptr(t), _nat.ptr(k), _nat.ptr(xe), _nat.ptr(tile_start), s)
        E_base, max_seqlen = meta.wait(dev)
        E = E_base * expand
        # exact-size copies of the event streams, so that callers that keep
        # them (autograd saves k and x_events for the backward) hold E
        # entries, not the worst case; the worst-case buffers are released
        # here (two small copy kernels, ~4E bytes each)
        k = k[:E].clone()
        if positions:
            ch, t = ch[:E].clone(), t[:E].clone()
        if xe is not None:
            xe = xe[:E].clone()
        return ch, t, k, cu, max_seqlen, xe, (bitmask, tile_start, expand)
