"""Drop-in for the flat_ch entry points of the reference extension module
`selective_scan_cuda` (csrc/selective_scan/selective_scan.cpp:674-1197),
backed by the HIP scan kernels of libbcm_event_scan.so.

fwd_flat_ch / bwd_flat_ch keep the reference's keyword names, defaults,
return lists and check messages. Implemented mode: depthwise B/C
(is_depthwise_bc=True, the only mode the BC_mamba block uses), with optional
D and z. The legacy [dstate, E] variable-B/C layout, the tiled layout and the
pointwise pw_B/pw_C mixing raise RuntimeError. The dense `fwd` / `bwd`
entry points of the reference module are not part of this build.
"""
import torch

try:
    from . import _native as _nat
except ImportError:  # imported with this directory on sys.path
    import _native as _nat

__all__ = ["fwd_flat_ch", "bwd_flat_ch"]

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def n_chunks_for(max_seqlen):
    """Chunk count of the saved state x: max(1, ceil(max_seqlen / 2048))."""
    return max(1, (int(max_seqlen) + 2047) // 2048)


def _common_checks(fn, u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D,
                   tile_offsets, is_depthwise_bc, pw_B, pw_C, extra_cuda=()):
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
    use_tiled = tile_offsets is not None
    if use_tiled or not is_depthwise_bc:
        raise RuntimeError(f"{fn}: only the depthwise B/C mode (is_depthwise_bc=True, no tile_offsets) "
                           "is implemented by the MI355X build")
    _check(B.dim() == 2 and C.dim() == 2, f"{fn} (depthwise): W_B/W_C must be 2-D [dim, dstate]")
    _check(tuple(B.shape) == (dim, dstate), f"{fn} (depthwise): W_B must be [dim, dstate]")
    _check(tuple(C.shape) == (dim, dstate), f"{fn} (depthwise): W_C must be [dim, dstate]")
    _check(B.is_contiguous() and C.is_contiguous(), f"{fn} (depthwise): W_B/W_C must be contiguous")
    if pw_B is not None or pw_C is not None:
        raise RuntimeError(f"{fn}: pointwise pw_B/pw_C mixing is not implemented by the MI355X build")
    if D is not None:
        _check(D.dtype == torch.float32, f"{fn}: D must be float32")
        _check(D.is_cuda and D.is_contiguous(), f"{fn}: D must be a contiguous CUDA tensor")
        _check(tuple(D.shape) == (dim,), f"{fn}: D must have shape ({dim},)")
    _check(int(max_seqlen) >= 0, f"{fn}: max_seqlen must be non-negative")
    return dim, dstate


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
    a.A, a.W_B, a.W_C = A.data_ptr(), B.data_ptr(), C.data_ptr()
    a.D = D.data_ptr() if D is not None else None
    a.z = z.data_ptr() if z is not None else None
    return a


def fwd_flat_ch(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D=None, z=None,
                tile_offsets=None, tile_chunk_size=0, is_depthwise_bc=False, pw_B=None, pw_C=None):
    """Flat per-channel scan forward -> [out, x] or [out, x, out_z]
    (selective_scan.cpp:674-884). x is [n_channels, n_chunks, 2*dstate]
    float32 holding, per 2048-event chunk and state, (prod of decays, h)."""
    fn = "selective_scan_fwd_flat_ch"
    _check(u_flat.is_contiguous() and k_flat.is_contiguous() and cu_seqlens.is_contiguous(),
           f"{fn}: u_flat/k_flat/cu_seqlens must be contiguous")
    _common_checks(fn, u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D,
                   tile_offsets, is_depthwise_bc, pw_B, pw_C)
    if z is not None:
        _check(z.dtype == u_flat.dtype, f"{fn}: z must have same dtype as u_flat")
        _check(z.is_cuda and z.is_contiguous(), f"{fn}: z must be a contiguous CUDA tensor")
        _check(z.dim() == 1 and z.size(0) == u_flat.size(0), f"{fn}: z must have shape (E,)")
    dev = u_flat.device
    n_ch = int(cu_seqlens.size(0)) - 1
    dstate = int(A.size(1))
    out = torch.empty_like(u_flat)
    x = torch.empty((n_ch, n_chunks_for(max_seqlen), dstate * 2), dtype=torch.float32, device=dev)
    out_z = torch.empty_like(u_flat) if z is not None else None
    a = _args(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle.contiguous(), dt_active.contiguous(),
              A.contiguous(), B, C, D, z)
    a.out, a.x = out.data_ptr(), x.data_ptr()
    a.out_z = out_z.data_ptr() if out_z is not None else None
    with torch.cuda.device(dev):
        _nat.call("bcm_scan_fwd", a, _nat.stream_of(u_flat))
    return [out, x] if z is None else [out, x, out_z]


def bwd_flat_ch(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, dout_flat, x,
                D=None, z=None, out=None, tile_offsets=None, tile_chunk_size=0, is_depthwise_bc=False,
                pw_B=None, pw_C=None):
    """Flat per-channel scan backward -> [du, dA, dW_B, dW_C, ddt_idle,
    ddt_active, (dD), (dz)] (selective_scan.cpp:890-1153). Parameter
    gradients are reduced deterministically inside the kernel."""
    fn = "selective_scan_bwd_flat_ch"
    _check(dout_flat.dtype == u_flat.dtype, f"{fn}: dout_flat must match u_flat dtype")
    _check(u_flat.is_contiguous() and k_flat.is_contiguous() and cu_seqlens.is_contiguous()
           and dout_flat.is_contiguous(), f"{fn}: u_flat/k_flat/cu_seqlens/dout_flat must be contiguous")
    _check(u_flat.dim() == 1 and k_flat.dim() == 1 and cu_seqlens.dim() == 1 and dout_flat.dim() == 1,
           f"{fn}: u_flat/k_flat/cu_seqlens/dout_flat must be 1-D")
    _check(dout_flat.size(0) == u_flat.size(0), f"{fn}: dout_flat must match u_flat shape")
    dim, dstate = _common_checks(fn, u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D,
                                 tile_offsets, is_depthwise_bc, pw_B, pw_C, extra_cuda=(dout_flat, x))
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
    f32 = dict(dtype=torch.float32, device=dev)
    du = torch.empty_like(u_flat)
    dA = torch.empty((dim, dstate), **f32)
    dW_B, dW_C = torch.empty((dim, dstate), **f32), torch.empty((dim, dstate), **f32)
    ddt_idle, ddt_active = torch.empty(dim, **f32), torch.empty(dim, **f32)
    dD = torch.empty(dim, **f32) if D is not None else None
    dz = torch.empty_like(u_flat) if has_z else None
    a = _args(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle.contiguous(), dt_active.contiguous(),
              A.contiguous(), B, C, D, z)
    a.dout, a.x_saved = dout_flat.data_ptr(), x.data_ptr()
    a.out_saved = out.data_ptr() if has_z else None
    a.du, a.dA, a.dW_B, a.dW_C = du.data_ptr(), dA.data_ptr(), dW_B.data_ptr(), dW_C.data_ptr()
    a.ddt_idle, a.ddt_active = ddt_idle.data_ptr(), ddt_active.data_ptr()
    a.dD = dD.data_ptr() if dD is not None else None
    a.dz = dz.data_ptr() if dz is not None else None
    with torch.cuda.device(dev):
        _nat.call("bcm_scan_bwd", a, _nat.stream_of(u_flat))
    res = [du, dA, dW_B, dW_C, ddt_idle, ddt_active]
    if D is not None:
        res.append(dD)
    if has_z:
        res.append(dz)
    return res
