"""Drop-in for the flat_ch part of the reference's
spike_mamba/selective_scan_interface.py (:1015-1237):
`SelectiveScanFlatChFn` and `selective_scan_flat_ch_fn`, same 16-slot
signature, same saved-tensor layout and backward slot order, calling the HIP
kernels through `selective_scan_cuda`.

Unlike the reference module, this one needs no `mamba_ssm` import.
`selective_scan_depthwise_bc_fn` is exported only so that `from
selective_scan_interface import selective_scan_flat_ch_fn,
selective_scan_depthwise_bc_fn` (e_model.py:83) resolves; the dense scans are
not part of this build and raise when called.
"""
import torch

try:
    from . import selective_scan_cuda
    from .runtime_breakdown import cuda_stage
except ImportError:  # imported with this directory on sys.path
    import selective_scan_cuda
    from runtime_breakdown import cuda_stage

__all__ = ["SelectiveScanFlatChFn", "selective_scan_flat_ch_fn", "selective_scan_depthwise_bc_fn"]


class SelectiveScanFlatChFn(torch.autograd.Function):
    """Autograd wrapper of fwd_flat_ch / bwd_flat_ch
    (selective_scan_interface.py:1015-1179).

    Forward input order: u_flat, k_flat, cu_seqlens, dt_idle, dt_active, A,
    B, C, D, z, max_seqlen, tile_offsets, tile_chunk_size, is_depthwise_bc,
    pw_B, pw_C. Returns (out, x) with out gated by silu(z) when z is given;
    x (per-chunk saved state) is not differentiable."""

    @staticmethod
    def forward(ctx, u_flat, k_flat, cu_seqlens, dt_idle, dt_active, A, B, C, D, z, max_seqlen,
                tile_offsets, tile_chunk_size, is_depthwise_bc, pw_B, pw_C):
        u_flat, k_flat, cu_seqlens = u_flat.contiguous(), k_flat.contiguous(), cu_seqlens.contiguous()
        dt_idle, dt_active = dt_idle.contiguous(), dt_active.contiguous()
        A, B, C = A.contiguous(), B.contiguous(), C.contiguous()
        if D is not None:
            D = D.contiguous()
        if z is not None:
            z = z.contiguous()
        if tile_offsets is not None:
            tile_offsets = tile_offsets.contiguous()
        if pw_B is not None:
            pw_B = pw_B.contiguous()
        if pw_C is not None:
            pw_C = pw_C.contiguous()
        chunk_g = acc = None
        if is_depthwise_bc and tile_offsets is None:
            chunk_g = selective_scan_cuda.chunk_states_buffer(u_flat, cu_seqlens, max_seqlen, A)
            # the per-event state sums, kept so the backward need not rebuild them
            acc = torch.empty(u_flat.shape, dtype=torch.float32, device=u_flat.device)
        result = selective_scan_cuda.fwd_flat_ch(
            u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C, D, z,
            tile_offsets, tile_chunk_size, is_depthwise_bc, pw_B, pw_C, _chunk_g=chunk_g, _acc=acc)
        # pass-start states and state sums for the backward (not autograd inputs)
        ctx.chunk_g, ctx.acc = chunk_g, acc
        out_flat, x = result[0], result[1]
        ctx.has_z, ctx.has_D, ctx.has_pw = z is not None, D is not None, pw_B is not None
        ctx.max_seqlen = max_seqlen
        ctx.tile_chunk_size = tile_chunk_size
        ctx.is_depthwise_bc = is_depthwise_bc
        saved = [u_flat, k_flat, cu_seqlens, dt_idle, dt_active, A, B, C, x]
        if ctx.has_D:
            saved.append(D)
        if ctx.has_z:
            saved.extend([z, out_flat])
        ctx.has_tile_offsets = tile_offsets is not None
        if tile_offsets is not None:
            saved.append(tile_offsets)
        if ctx.has_pw:
            saved.extend([pw_B, pw_C])
        ctx.save_for_backward(*saved)
        ctx.mark_non_differentiable(x)
        # x has no gradient: autograd passes None for it instead of a zero
        # tensor (and None for out when the graph does not use it)
        ctx.set_materialize_grads(False)
        ctx.out_meta = (u_flat.shape, u_flat.dtype, u_flat.device)
        return (result[2] if ctx.has_z else out_flat), x

    @staticmethod
    def backward(ctx, dout, _dx):
        if dout is None:
            shape, dtype, dev = ctx.out_meta
            dout = torch.zeros(shape, dtype=dtype, device=dev)
        if dout.stride(-1) != 1:
            dout = dout.contiguous()
        saved = list(ctx.saved_tensors)
        u_flat, k_flat, cu_seqlens, dt_idle, dt_active, A, B, C, x = saved[:9]
        idx = 9
        D = z = out_flat = tile_offsets = pw_B = pw_C = None
        if ctx.has_D:
            D = saved[idx]
            idx += 1
        if ctx.has_z:
            z, out_flat = saved[idx], saved[idx + 1]
            idx += 2
        if ctx.has_tile_offsets:
            tile_offsets = saved[idx]
            idx += 1
        if ctx.has_pw:
            pw_B, pw_C = saved[idx], saved[idx + 1]
        with cuda_stage("sparse_scan_backward"):
            result = selective_scan_cuda.bwd_flat_ch(
                u_flat, k_flat, cu_seqlens, ctx.max_seqlen, dt_idle, dt_active, A, B, C, dout.contiguous(), x,
                D, z, out_flat, tile_offsets, ctx.tile_chunk_size, ctx.is_depthwise_bc, pw_B, pw_C,
                _chunk_g=ctx.chunk_g, _trusted_seqlen=True, _acc=ctx.acc)  # the forward checked max_seqlen
        du, dA, dW_B, dW_C, ddt_idle, ddt_active = result[:6]
        ridx = 6
        dD = dz = dpw_B = dpw_C = None
        if ctx.has_D:
            dD = result[ridx]
            ridx += 1
        if ctx.has_z:
            dz = result[ridx]
            ridx += 1
        if ctx.has_pw:
            dpw_B, dpw_C = result[ridx], result[ridx + 1]
        return (du, None, None, ddt_idle, ddt_active, dA, dW_B, dW_C, dD, dz,
                None, None, None, None, dpw_B, dpw_C)


def selective_scan_flat_ch_fn(u_flat, k_flat, cu_seqlens, max_seqlen, dt_idle, dt_active, A, B, C,
                              D=None, z=None, tile_offsets=None, tile_chunk_size=0, is_depthwise_bc=False,
                              pw_B=None, pw_C=None):
    """Autograd-enabled flat per-channel selective scan
    (selective_scan_interface.py:1182-1237). In depthwise mode B and C are
    the [dim, dstate] weights W_B / W_C; B[i,s] = u[i]*W_B[d,s] and
    C[i,s] = u[i]*W_C[d,s] are formed in the kernel. Returns (out, x)."""
    u_flat, k_flat, cu_seqlens = u_flat.contiguous(), k_flat.contiguous(), cu_seqlens.contiguous()
    dt_idle, dt_active = dt_idle.contiguous(), dt_active.contiguous()
    A, B, C = A.contiguous(), B.contiguous(), C.contiguous()
    if D is not None:
        D = D.contiguous()
    if z is not None:
        z = z.contiguous()
    if tile_offsets is not None:
        tile_offsets = tile_offsets.contiguous()
    if pw_B is not None:
        pw_B = pw_B.contiguous()
    if pw_C is not None:
        pw_C = pw_C.contiguous()
    return SelectiveScanFlatChFn.apply(u_flat, k_flat, cu_seqlens, dt_idle, dt_active, A, B, C, D, z, max_seqlen,
                                       tile_offsets, tile_chunk_size, is_depthwise_bc, pw_B, pw_C)


def selective_scan_depthwise_bc_fn(*args, **kwargs):
    """Dense depthwise scan of the reference module (:618-688); not on the
    event path and not part of this build."""
    raise RuntimeError("selective_scan_depthwise_bc_fn: the dense scan is not part of the MI355X event-path build")
