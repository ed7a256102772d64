"""Drop-in for the flat_ch entry points of the reference extension module
`selective_scan_cuda` (csrc/selective_scan/selective_scan.cpp:674-1197),
backed by the HIP scan kernels of libbcm_event_scan.so.

fwd_flat_ch / bwd_flat_ch keep the reference's keyword names, defaults,
return lists and check messages, in every B/C mode the reference accepts:
  depthwise (is_depthwise_bc=True)  B, C = W_B, W_C [dim, dstate]; the
      BC_mamba block's mode, on the tuned kernels bcm_scan_fwd / _bwd;
  depthwise + pointwise (pw_B, pw_C [dim, dim])  the scan runs on
      W_eff = pw @ W (selective_scan_fwd_kernel.cuh:486-509) and the
      backward maps dW_eff to dW = pw^T dW_eff and dpw = dW_eff W^T
      (selective_scan_bwd_kernel.cuh:1122-1166); the two small products are
      plain library GEMMs;
  legacy (is_depthwise_bc=False)  B, C [dstate, E] per event (the backward
      also takes [dstate, dim] per model channel);
  tiled (tile_offsets given)  B, C [n_tiles, dstate, tile_chunk_size];
the last two on bcm_scan_var_fwd / _bwd. The dense `fwd` / `bwd` entry
points of the reference module are not part of this build.
"""
import torch

try:
    from . import _native as _nat
    from . import _provenance as _prov
except ImportError:  # imported with this directory on sys.path
    import _native as _nat
    import _provenance as _prov

__all__ = ["fwd_flat_ch", "bwd_flat_ch"]

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def n_chunks_for(max_seqlen):
    """Chunk count of the saved state x: max(1, ceil(max_seqlen / 2048))."""
    return max(1, (int(max_seqlen) + 2047) // 2048)


def _common_checks(fn, u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D,
                   tile_offsets, is_depthwise_bc, pw_B, pw_C, extra_cuda=(), bwd=False, tile_chunk_size=0):
    """The reference's checks (selective_scan.cpp:697-781, 939-998); returns
    (dim, dstate, mode) with mode "depthwise", "tiled" or "legacy"."""
    _check(u_flat.dtype in _FLOATS, f"{fn}: u_flat must be fp16/bf16/fp32")
    _check(A.dtype == torch.float32, f"{fn}: A must be float32")
    _check(B.dtype == torch.float32, f"{fn}: B must be float32")
    _check(C.dtype == torch.float32, f"{fn}: C must be float32")
    _check(all(t.is_cuda for t in (u_flat, k_flat, cu_seqlens, dt_idle, dt_active, A, B, C, *extra_cuda)),
           f"{fn}: all tensors must be CUDA tensors")
    _check(u_flat.dim() == 1, f"{fn}: u_flat must be 1-D")
    _check(k_flat.dim() == 1, f"{fn}: k_flat must be 1-D")
    _check(cu_seqlens.dim() == 1, f"{fn}: cu_seqlens must be 1-D")
    _check(k_flat.dtype == torch.int32, f"{fn}: k_flat must be int32")
    _check(cu_seqlens.dtype == torch.int32, f"{fn}: cu_seqlens must be int32")
    _check(k_flat.size(0) == u_flat.size(0), f"{fn}: k_flat must match u_flat shape")
    _check(cu_seqlens.size(0) >= 2, f"{fn}: cu_seqlens must have at least 2 elements")
    _check(dt_idle.dtype == torch.float32 and dt_active.dtype == torch.float32,
           f"{fn}: dt_idle/dt_active must be float32")
    _check(dt_idle.dim() == 1 and dt_active.dim() == 1, f"{fn}: dt_idle/dt_active must be 1-D")
    _check(A.dim() == 2, f"{fn}: A must be 2-D (dim, dstate)")
    dim, dstate = A.shape
    _check(dstate <= 256, f"{fn}: dstate must be <= 256")
    _check(tuple(dt_idle.shape) == (dim,), f"{fn}: dt_idle must have shape ({dim},)")
    _check(tuple(dt_active.shape) == (dim,), f"{fn}: dt_active must have shape ({dim},)")
    E = int(u_flat.size(0))
    use_tiled = tile_offsets is not None
    if is_depthwise_bc and not use_tiled:
        _check(B.dim() == 2 and C.dim() == 2, f"{fn} (depthwise): W_B/W_C must be 2-D [dim, dstate]")
        _check(tuple(B.shape) == (dim, dstate), f"{fn} (depthwise): W_B must be [dim, dstate]")
        _check(tuple(C.shape) == (dim, dstate), f"{fn} (depthwise): W_C must be [dim, dstate]")
        _check(B.is_contiguous() and C.is_contiguous(), f"{fn} (depthwise): W_B/W_C must be contiguous")
        if pw_B is not None:
            _check(pw_C is not None, f"{fn}: pw_C is required with pw_B")
            _check(pw_B.dtype == torch.float32 and pw_C.dtype == torch.float32, f"{fn}: pw_B/pw_C must be float32")
            _check(pw_B.is_cuda and pw_C.is_cuda and pw_B.is_contiguous() and pw_C.is_contiguous(),
                   f"{fn}: pw_B/pw_C must be CUDA and contiguous")
            _check(pw_B.dim() == 2 and tuple(pw_B.shape) == (dim, dim), f"{fn}: pw_B must be [dim, dim]")
            _check(pw_C.dim() == 2 and tuple(pw_C.shape) == (dim, dim), f"{fn}: pw_C must be [dim, dim]")
        mode = "depthwise"
    elif use_tiled:
        _check(B.dim() == 3 and C.dim() == 3, f"{fn}: tiled B/C must be 3-D [N_tiles, dstate, tile_chunk_size]")
        _check(B.size(1) == dstate and C.size(1) == dstate, f"{fn}: tiled B/C dim-1 must equal dstate")
        _check(B.is_contiguous() and C.is_contiguous(), f"{fn}: tiled B/C must be contiguous")
        _check(int(tile_chunk_size) >= 1 and B.size(2) == int(tile_chunk_size) and C.size(2) == int(tile_chunk_size),
               f"{fn}: tiled B/C dim-2 must equal tile_chunk_size (>= 1)")
        _check(B.size(0) == C.size(0), f"{fn}: tiled B and C must have the same number of tiles")
        _check(tile_offsets.is_cuda and tile_offsets.dtype == torch.int32 and tile_offsets.dim() == 1
               and tile_offsets.is_contiguous() and tile_offsets.size(0) >= cu_seqlens.size(0) - 1,
               f"{fn}: tile_offsets must be a contiguous int32 CUDA tensor with one entry per channel")
        mode = "tiled"
    else:
        if not bwd:
            _check(B.dim() == 2 and C.dim() == 2, f"{fn}: B/C must be 2-D (dstate, E) [transposed layout]")
            _check(tuple(B.shape) == (dstate, E), f"{fn}: B must have shape ({dstate}, {E})")
            _check(tuple(C.shape) == (dstate, E), f"{fn}: C must have shape ({dstate}, {E})")
            _check(B.stride(1) == 1 and C.stride(1) == 1,
                   f"{fn}: B/C must have contiguous last dimension (stride(1) == 1)")
        else:
            _check(B.dim() == 2 and C.dim() == 2, f"{fn}: B/C must be 2-D [dstate, E] or [dstate, dim]")
            _check(B.stride(1) == 1 and C.stride(1) == 1, f"{fn}: B/C must have contiguous last dimension")
            for name, t in (("B", B), ("C", C)):
                _check(t.size(0) == dstate and t.size(1) in (E, dim),
                       f"{fn}: {name} must have shape ({dstate}, {E}) or ({dstate}, {dim})")
        mode = "legacy"
    if D is not None:
        _check(D.dtype == torch.float32, f"{fn}: D must be float32")
        _check(D.is_cuda and D.is_contiguous(), f"{fn}: D must be a contiguous CUDA tensor")
        _check(tuple(D.shape) == (dim,), f"{fn}: D must have shape ({dim},)")
    _check(int(max_seqlen) >= 0, f"{fn}: max_seqlen must be non-negative")
    return dim, dstate, mode


class _SeqlenStatus:
    """The scan kernels' status word (bcm_scan_args.status) for a call whose
    max_seqlen comes from the caller: zeroed before the launch, read after
    it (one host sync), RuntimeError when some channel held more than
    max_seqlen events (its saved states would be incomplete)."""

    def __init__(self, fn, max_seqlen, dev, enabled):
        self.fn, self.max_seqlen = fn, int(max_seqlen)
        self.t = torch.zeros(1, dtype=torch.int32, device=dev) if enabled else None

    def attach(self, a):
        a.status = self.t.data_ptr() if self.t is not None else None

    def check(self):
        v = int(self.t.item()) if self.t is not None else 0
        if v == _nat.SCAN_SEQLEN_EXCEEDED:
            raise RuntimeError(f"{self.fn}: a channel holds more than max_seqlen = {self.max_seqlen} events "
                               "(cu_seqlens and max_seqlen disagree)")
        if v == _nat.SCAN_ROWS_INCOMPLETE:
            raise RuntimeError(f"{self.fn}: the dense gradient rows are incomplete (a row writer stopped waiting "
                               "for the scan)")


def _needs_report(trusted, n_ch, cu_seqlens, max_seqlen):
    """Whether a call reads the kernels' length report: not for callers that
    computed max_seqlen themselves, nor for offsets whose longest channel the
    extraction recorded (bc_mamba_amd._provenance) and max_seqlen covers."""
    return not trusted and n_ch > 0 and not _prov.covers_max_seqlen(cu_seqlens, max_seqlen)


def _acc_ptr(fn, acc, u_flat):
    """Device pointer of a per-event state-sum buffer (float32 [E]), or None."""
    if acc is None:
        return None
    _check(acc.dtype == torch.float32 and acc.is_contiguous() and acc.numel() == u_flat.numel()
           and acc.device == u_flat.device, f"{fn}: _acc must be a contiguous float32 (E,) tensor on u's device")
    return acc.data_ptr()


def _bc(mode, B, C, E, tile_offsets, tile_chunk_size, dB=None, dC=None):
    """bcm_scan_bc of the legacy / tiled modes. Legacy B/C are per event when
    their second dimension is E, else per model channel, as
    set_ssm_params_flat_seg_fwd decides (selective_scan.cpp:304-305)."""
    bc = _nat.ScanBC()
    bc.B, bc.C = B.data_ptr(), C.data_ptr()
    if mode == "tiled":
        bc.layout = _nat.BC_TILED
        bc.b_per_event = bc.c_per_event = 1
        bc.tile_chunk_size = int(tile_chunk_size)
        bc.n_tiles = int(B.size(0))
        bc.tile_offsets = tile_offsets.data_ptr()
    else:
        bc.layout = _nat.BC_LEGACY
        bc.b_per_event = int(B.size(1) == E)
        bc.c_per_event = int(C.size(1) == E)
        bc.b_row_stride, bc.c_row_stride = int(B.stride(0)), int(C.stride(0))
    if dB is not None:
        bc.dB, bc.dC = dB.data_ptr(), dC.data_ptr()
        if mode == "legacy":
            bc.db_row_stride, bc.dc_row_stride = int(dB.stride(0)), int(dC.stride(0))
    return bc


def chunk_states_buffer(u_flat, cu_seqlens, max_seqlen, A):
    """float32 [n_channels, n_pass, dstate] buffer for the depthwise scan's
    pass-start states h, or None when every channel fits one pass (or passes
    are 2048 events, which re-seed from x)."""
    a = _nat.ScanArgs()
    a.n_events = int(u_flat.size(0))
    a.n_channels = int(cu_seqlens.size(0)) - 1
    a.dim, a.dstate = int(A.size(0)), int(A.size(1))
    a.max_seqlen = int(max_seqlen)
    pass_len, n_pass, needs = _nat.scan_chunking(a)
    if not needs:
        return None
    buf = torch.empty((a.n_channels, n_pass, a.dstate), dtype=torch.float32, device=u_flat.device)
    buf.bcm_pass_len = pass_len  # checked by the kernels against their own passes (chunk_g_pass)
    return buf


def _args(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D, z):
    dim, dstate = A.shape
    a = _nat.ScanArgs()
    a.n_events = int(u_flat.size(0))
    a.n_channels = int(cu_seqlens.size(0)) - 1
    a.dim, a.dstate = int(dim), int(dstate)
    a.max_seqlen = int(max_seqlen)
    a.n_chunks = n_chunks_for(max_seqlen)
    a.dtype = _nat.dtype_code(u_flat.dtype)
    a.u, a.k, a.cu_seqlens = u_flat.data_ptr(), k_flat.data_ptr(), cu_seqlens.data_ptr()
    a.dt_idle, a.dt_active = dt_idle.data_ptr(), dt_active.data_ptr()
    a.A = A.data_ptr()
    a.W_B = B.data_ptr() if B is not None else None
    a.W_C = C.data_ptr() if C is not None else None
    a.D = D.data_ptr() if D is not None else None
    a.z = z.data_ptr() if z is not None else None
    return a


def fwd_flat_ch(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D=None, z=None,
                tile_offsets=None, tile_chunk_size=0, is_depthwise_bc=False, pw_B=None, pw_C=None, _chunk_g=None,
                _trusted_seqlen=False, _acc=None):
    """Flat per-channel scan forward -> [out, x] or [out, x, out_z]
    (selective_scan.cpp:674-884). x is [n_channels, n_chunks, 2*dstate]
    float32 holding, per 2048-event chunk and state, (prod of decays, h).
    `_chunk_g` (not in the reference signature): a float32 tensor from
    chunk_states_buffer() that receives the pass-start states, so that
    bwd_flat_ch need not recompute them (depthwise mode). `_acc` (not in the
    reference signature either): a float32 [E] tensor that receives the
    per-event state sums Σ_s W_B W_C h/W_B, which bwd_flat_ch(_acc=...) then
    reads instead of rebuilding them (depthwise mode).
    In depthwise mode the kernels report a channel longer than max_seqlen
    and this call raises RuntimeError (one host sync to read the report);
    `_trusted_seqlen=True` skips the report for callers whose max_seqlen
    comes from the extraction itself; so does a cu_seqlens returned by this
    package's extraction (unchanged) with a max_seqlen at least its longest
    channel, which the extraction recorded on it."""
    fn = "selective_scan_fwd_flat_ch"
    _check(u_flat.is_contiguous() and k_flat.is_contiguous() and cu_seqlens.is_contiguous(),
           f"{fn}: u_flat/k_flat/cu_seqlens must be contiguous")
    _, dstate, mode = _common_checks(fn, u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D,
                                     tile_offsets, is_depthwise_bc, pw_B, pw_C, tile_chunk_size=tile_chunk_size)
    if z is not None:
        _check(z.dtype == u_flat.dtype, f"{fn}: z must have same dtype as u_flat")
        _check(z.is_cuda and z.is_contiguous(), f"{fn}: z must be a contiguous CUDA tensor")
        _check(z.dim() == 1 and z.size(0) == u_flat.size(0), f"{fn}: z must have shape (E,)")
    dev = u_flat.device
    n_ch = int(cu_seqlens.size(0)) - 1
    out = torch.empty_like(u_flat)
    x = torch.empty((n_ch, n_chunks_for(max_seqlen), dstate * 2), dtype=torch.float32, device=dev)
    out_z = torch.empty_like(u_flat) if z is not None else None
    with torch.cuda.device(dev):
        if mode == "depthwise" and pw_B is not None:
            B, C = pw_B @ B, pw_C @ C  # W_eff [dim, dstate]
        a = _args(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle.contiguous(), dt_active.contiguous(),
                  A.contiguous(), B if mode == "depthwise" else None, C if mode == "depthwise" else None, D, z)
        a.out, a.x = out.data_ptr(), x.data_ptr()
        a.out_z = out_z.data_ptr() if out_z is not None else None
        if mode == "depthwise":
            _nat.attach_chunk_g(a, _chunk_g)
            a.acc = _acc_ptr(fn, _acc, u_flat)
            status = _SeqlenStatus(fn, max_seqlen, dev, _needs_report(_trusted_seqlen, n_ch, cu_seqlens, max_seqlen))
            status.attach(a)
            _nat.call("bcm_scan_fwd", a, _nat.stream_of(u_flat))
            status.check()
        else:
            bc = _bc(mode, B, C, int(u_flat.size(0)), tile_offsets, tile_chunk_size)
            _nat.call("bcm_scan_var_fwd", a, bc, _nat.stream_of(u_flat))
    return [out, x] if z is None else [out, x, out_z]


def bwd_flat_ch(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, dout_flat, x,
                D=None, z=None, out=None, tile_offsets=None, tile_chunk_size=0, is_depthwise_bc=False,
                pw_B=None, pw_C=None, _chunk_g=None, _rows=None, _trusted_seqlen=False, _acc=None,
                _discard_du=False):
    """Flat per-channel scan backward -> [du, dA, dB, dC, ddt_idle,
    ddt_active, (dD), (dz), (dpw_B, dpw_C)] (selective_scan.cpp:890-1153).
    dB / dC are dW_B / dW_C [dim, dstate] in depthwise mode and have the
    shape of B / C otherwise. Parameter gradients are reduced
    deterministically inside the kernels.
    `_rows` (not in the reference signature; depthwise mode without pw_B):
    (bitmask, mask_row_div, tile_start, dx) of the extraction's event index
    and a contiguous [n_channels, L] tensor of u_flat's dtype, which also
    receives the gather backward of du (du at the events, 0 elsewhere).
    `_acc`: the per-event state sums a fwd_flat_ch(_acc=...) of the same
    inputs wrote (depthwise mode), read instead of rebuilt.
    `_discard_du` (with `_rows`): a caller that needs only dx; where the
    scan kernel writes the rows itself, du is not stored and the result's
    du slot is None (dx holds the same values at the events).
    As fwd_flat_ch, raises RuntimeError when a channel holds more than
    max_seqlen events (unless `_trusted_seqlen`)."""
    fn = "selective_scan_bwd_flat_ch"
    _check(dout_flat.dtype == u_flat.dtype, f"{fn}: dout_flat must match u_flat dtype")
    _check(u_flat.is_contiguous() and k_flat.is_contiguous() and cu_seqlens.is_contiguous()
           and dout_flat.is_contiguous(), f"{fn}: u_flat/k_flat/cu_seqlens/dout_flat must be contiguous")
    _check(u_flat.dim() == 1 and k_flat.dim() == 1 and cu_seqlens.dim() == 1 and dout_flat.dim() == 1,
           f"{fn}: u_flat/k_flat/cu_seqlens/dout_flat must be 1-D")
    _check(dout_flat.size(0) == u_flat.size(0), f"{fn}: dout_flat must match u_flat shape")
    dim, dstate, mode = _common_checks(fn, u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D,
                                       tile_offsets, is_depthwise_bc, pw_B, pw_C, extra_cuda=(dout_flat, x),
                                       bwd=True, tile_chunk_size=tile_chunk_size)
    n_ch = int(cu_seqlens.size(0)) - 1
    _check(x.dtype == torch.float32, f"{fn}: x must be float32")
    _check(x.is_contiguous(), f"{fn}: x must be contiguous")
    _check(x.dim() == 3 and x.size(0) == n_ch and x.size(2) == dstate * 2,
           f"{fn}: x must have shape (n_channels, n_chunks, dstate*2)")
    _check(x.size(1) == n_chunks_for(max_seqlen),
           f"{fn}: x.size(1) must equal n_chunks = (max_seqlen + 2047) / 2048")
    has_z = z is not None
    if has_z:
        _check(out is not None, f"{fn}: out (forward ungated output) must be provided when z is provided")
        _check(z.dtype == u_flat.dtype and out.dtype == u_flat.dtype, f"{fn}: z/out must match u_flat dtype")
        _check(z.is_cuda and out.is_cuda and z.is_contiguous() and out.is_contiguous(),
               f"{fn}: z/out must be contiguous CUDA tensors")
        _check(z.size(0) == u_flat.size(0) and out.size(0) == u_flat.size(0), f"{fn}: z/out must have shape (E,)")
    dev = u_flat.device
    E = int(u_flat.size(0))
    f32 = dict(dtype=torch.float32, device=dev)
    du = torch.empty_like(u_flat)
    dA = torch.empty((dim, dstate), **f32)
    ddt_idle, ddt_active = torch.empty(dim, **f32), torch.empty(dim, **f32)
    dD = torch.empty(dim, **f32) if D is not None else None
    dz = torch.empty_like(u_flat) if has_z else None
    dpw_B = dpw_C = None
    with torch.cuda.device(dev):
        s = _nat.stream_of(u_flat)
        if mode == "depthwise":
            W_B, W_C = (pw_B @ B, pw_C @ C) if pw_B is not None else (B, C)
            dB, dC = torch.empty((dim, dstate), **f32), torch.empty((dim, dstate), **f32)
        else:
            W_B = W_C = None
            # tiled entries that no event maps to stay zero (the reference
            # zero-fills and accumulates, :1055-1056)
            dB = torch.zeros(B.shape, **f32) if mode == "tiled" else torch.empty(B.shape, **f32)
            dC = torch.zeros(C.shape, **f32) if mode == "tiled" else torch.empty(C.shape, **f32)
        a = _args(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle.contiguous(), dt_active.contiguous(),
                  A.contiguous(), W_B, W_C, D, z)
        a.dout, a.x_saved = dout_flat.data_ptr(), x.data_ptr()
        a.out_saved = out.data_ptr() if has_z else None
        a.du, a.dA = du.data_ptr(), dA.data_ptr()
        a.ddt_idle, a.ddt_active = ddt_idle.data_ptr(), ddt_active.data_ptr()
        a.dD = dD.data_ptr() if dD is not None else None
        a.dz = dz.data_ptr() if dz is not None else None
        if mode == "depthwise":
            status = _SeqlenStatus(fn, max_seqlen, dev, _needs_report(_trusted_seqlen, n_ch, cu_seqlens, max_seqlen))
            status.attach(a)
            a.dW_B, a.dW_C = dB.data_ptr(), dC.data_ptr()
            _, _, needs_g = _nat.scan_chunking(a)
            if needs_g and _chunk_g is None:
                # passes shorter than 2048 events start from the forward's
                # pass states: recompute them with a forward run
                _chunk_g = chunk_states_buffer(u_flat, cu_seqlens, max_seqlen, A)
                f = _args(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle.contiguous(), dt_active.contiguous(),
                          A.contiguous(), W_B, W_C, D, z)
                scratch_out = torch.empty_like(u_flat)
                f.out, f.x = scratch_out.data_ptr(), torch.empty_like(x).data_ptr()
                f.out_z = torch.empty_like(u_flat).data_ptr() if has_z else None
                _nat.attach_chunk_g(f, _chunk_g)
                status.attach(f)
                _nat.call("bcm_scan_fwd", f, s)
            _nat.attach_chunk_g(a, _chunk_g)
            a.acc = _acc_ptr(fn, _acc, u_flat)
            split_bytes = int(_nat.lib().bcm_scan_bwd_workspace_bytes(a))
            split_ws = torch.empty(split_bytes // 4, dtype=torch.float32, device=dev) if split_bytes else None
            a.split_ws = split_ws.data_ptr() if split_ws is not None else None
            a.split_ws_bytes = split_bytes
            if _rows is None:
                _nat.call("bcm_scan_bwd", a, s)
            else:
                bitmask, mrd, tile_start, dx = _rows
                _check(pw_B is None, f"{fn}: dense rows need W_B / W_C without pw_B / pw_C")
                _check(dx.is_contiguous() and dx.dtype == u_flat.dtype and dx.dim() == 2
                       and dx.size(0) == n_ch, f"{fn}: dx must be a contiguous (n_channels, L) tensor of u's dtype")
                r = _nat.ScanRows()
                r.bitmask, r.mask_row_div, r.tile_start = bitmask.data_ptr(), int(mrd), tile_start.data_ptr()
                r.seqlen, r.dx = int(dx.size(1)), dx.data_ptr()
                if _discard_du and _nat.lib().bcm_scan_bwd_rows_fused(a, r) == 1:
                    a.du, du = None, None
                _nat.call("bcm_scan_bwd_rows", a, r, s)
            status.check()
            if pw_B is not None:  # dB, dC hold dW_eff here
                dpw_B, dpw_C = dB @ B.t(), dC @ C.t()
                dB, dC = pw_B.t() @ dB, pw_C.t() @ dC
        else:
            bc = _bc(mode, B, C, E, tile_offsets, tile_chunk_size, dB, dC)
            nbytes = int(_nat.lib().bcm_scan_var_workspace_bytes(E, dstate))
            ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=dev)
            _nat.call("bcm_scan_var_bwd", a, bc, ws.data_ptr(), nbytes, s)
    res = [du, dA, dB, dC, ddt_idle, ddt_active]
    if D is not None:
        res.append(dD)
    if has_z:
        res.append(dz)
    if dpw_B is not None:
        res.extend([dpw_B, dpw_C])
    return res
