"""ctypes binding of libbcm_event_scan.so, the C ABI declared in
include/bcm_event_scan.h.

torch is imported first on purpose: the library links the HIP runtime by
SONAME, so loading it after torch binds it to the runtime torch already uses
(one set of streams, one device-pointer space). There is no CPU fallback:
if the library is missing, every entry point raises.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("BCM_LIB_PATH", os.path.join(_HERE, "lib", "libbcm_event_scan.so"))

F32, F16, BF16, U8 = 0, 1, 2, 3
ABI_VERSION = 4  # BCM_ABI_VERSION of include/bcm_event_scan.h
_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.bool: U8, torch.uint8: U8}

c_i32, c_i64, c_f32, c_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class ScanArgs(ctypes.Structure):
    """Mirror of bcm_scan_args (field order and types must match the header)."""

    _fields_ = [
        ("n_events", c_i64), ("n_channels", c_i32), ("dim", c_i32), ("dstate", c_i32),
        ("max_seqlen", c_i32), ("n_chunks", c_i32), ("dtype", c_i32),
        ("u", c_p), ("k", c_p), ("cu_seqlens", c_p), ("dt_idle", c_p), ("dt_active", c_p),
        ("A", c_p), ("W_B", c_p), ("W_C", c_p), ("D", c_p), ("z", c_p),
        ("out", c_p), ("out_z", c_p), ("x", c_p),
        ("dout", c_p), ("x_saved", c_p), ("out_saved", c_p),
        ("du", c_p), ("dA", c_p), ("dW_B", c_p), ("dW_C", c_p), ("ddt_idle", c_p),
        ("ddt_active", c_p), ("dD", c_p), ("dz", c_p), ("chunk_g", c_p), ("chunk_g_bytes", c_i64),
        ("split_ws", c_p), ("split_ws_bytes", c_i64), ("status", c_p), ("chunk_g_pass", c_i32),
        ("acc", c_p),
    ]


SCAN_SEQLEN_EXCEEDED = 1  # bcm_scan_args.status: a channel holds more than max_seqlen events
SCAN_ROWS_INCOMPLETE = 2  # bcm_scan_args.status: bcm_scan_bwd_rows left the dense rows incomplete


class ScanRows(ctypes.Structure):
    """Mirror of bcm_scan_rows (field order and types must match the header)."""

    _fields_ = [("bitmask", c_p), ("mask_row_div", c_i64), ("tile_start", c_p), ("seqlen", c_i64), ("dx", c_p)]


class ScanBC(ctypes.Structure):
    """Mirror of bcm_scan_bc (field order and types must match the header)."""

    _fields_ = [
        ("layout", c_i32), ("b_per_event", c_i32), ("c_per_event", c_i32), ("tile_chunk_size", c_i32),
        ("b_row_stride", c_i64), ("c_row_stride", c_i64), ("n_tiles", c_i64),
        ("tile_offsets", c_p), ("B", c_p), ("C", c_p), ("dB", c_p), ("dC", c_p),
        ("db_row_stride", c_i64), ("dc_row_stride", c_i64),
    ]


BC_LEGACY, BC_TILED = 1, 2

# name -> (restype, argtypes); exactly the functions declared in the header.
SIGNATURES = {
    "bcm_abi_version": (c_i32, []),
    "bcm_last_error": (ctypes.c_char_p, []),
    "bcm_bitmask_words": (c_i64, [c_i64]),
    "bcm_tile_count": (c_i64, [c_i64]),
    "bcm_zero": (c_i32, [c_p, c_i64, c_p]),
    "bcm_extract_count": (c_i32, [c_p, c_i32, c_i64, c_i64, c_f32, c_p, c_p, c_p]),
    "bcm_extract_scan": (c_i32, [c_p, c_i64, c_p, c_p, c_p]),
    "bcm_extract_fill": (c_i32, [c_p, c_p, c_i64, c_i64, c_i64, c_p, c_i32, c_p, c_p, c_p, c_p, c_p, c_p, c_p]),
    "bcm_extract_block_sums_bytes": (c_i64, [c_i64]),
    "bcm_extract_count_blocks": (c_i32, [c_p, c_i32, c_i64, c_i64, c_f32, c_p, c_p, c_p, c_p]),
    "bcm_extract_fill_blocks": (c_i32, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_p, c_i32, c_p, c_p, c_p, c_p,
                                        c_p, c_p, c_p]),
    "bcm_expand_events": (c_i32, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_p, c_p, c_p, c_p, c_p]),
    "bcm_seqlen_max": (c_i32, [c_p, c_i64, c_p, c_p]),
    "bcm_gather_fwd": (c_i32, [c_p, c_i32, c_i64, c_i64, c_p, c_p, c_i64, c_p, c_p]),
    "bcm_gather_bwd": (c_i32, [c_p, c_i32, c_p, c_p, c_i64, c_i64, c_i64, c_p, c_p]),
    "bcm_gather_bwd_rows": (c_i32, [c_p, c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_p, c_p]),
    "bcm_scan_fwd": (c_i32, [ctypes.POINTER(ScanArgs), c_p]),
    "bcm_scan_bwd": (c_i32, [ctypes.POINTER(ScanArgs), c_p]),
    "bcm_scan_bwd_rows": (c_i32, [ctypes.POINTER(ScanArgs), ctypes.POINTER(ScanRows), c_p]),
    "bcm_scan_bwd_rows_fused": (c_i32, [ctypes.POINTER(ScanArgs), ctypes.POINTER(ScanRows)]),
    "bcm_scan_bwd_workspace_bytes": (c_i64, [ctypes.POINTER(ScanArgs)]),
    "bcm_set_scan_family": (c_i32, [c_i32]),
    "bcm_scan_chunking": (c_i32, [ctypes.POINTER(ScanArgs), ctypes.POINTER(c_i32), ctypes.POINTER(c_i32),
                                  ctypes.POINTER(c_i32)]),
    "bcm_scan_var_fwd": (c_i32, [ctypes.POINTER(ScanArgs), ctypes.POINTER(ScanBC), c_p]),
    "bcm_scan_var_workspace_bytes": (c_i64, [c_i64, c_i32]),
    "bcm_scan_var_bwd": (c_i32, [ctypes.POINTER(ScanArgs), ctypes.POINTER(ScanBC), c_p, c_i64, c_p]),
    "bcm_spike_bits": (c_i32, [c_p, c_i32, c_i64, c_i64, c_i64, ctypes.c_float, c_p, c_p, c_p]),
    "bcm_extract_count_bits": (c_i32, [c_p, c_i64, c_i64, c_p, c_p, c_p]),
    "bcm_extract_fill_blocks_conv": (c_i32, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_p, c_i32, c_i64, c_i64, c_i64,
                                             c_p, c_p, c_i32, c_i32, c_p, c_p, c_p, c_p, c_p, c_p, c_p]),
    "bcm_causal_conv1d_bwd_events_workspace_bytes": (c_i64, [c_i64, c_i64, c_i32]),
    "bcm_causal_conv1d_bwd_events": (c_i32, [c_p, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_p, c_p, c_i32, c_i32,
                                             c_p, c_i64, c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_i64, c_p]),
    "bcm_causal_conv1d_fwd": (c_i32, [c_p, c_i32, c_p, c_p, c_i64, c_i64, c_i64, c_i32, c_i32, c_p, c_p]),
    "bcm_causal_conv1d_bwd_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i32]),
    "bcm_causal_conv1d_bwd": (c_i32, [c_p, c_i32, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i32, c_i32, c_p, c_p, c_p,
                                      c_p, c_i64, c_p]),
    "bcm_build_event_index": (c_i32, [c_p, c_p, c_i64, c_i64, c_p, c_p, c_p, c_i64, c_p]),
    "bcm_restore_fwd": (c_i32, [c_p, c_i32, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_i32, c_p]),
    "bcm_restore_bwd_workspace_bytes": (c_i64, [c_i64, c_i64]),
    "bcm_restore_bwd": (c_i32, [c_p, c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_i64, c_p, c_i64, c_p]),
    "bcm_restore_bwd_noalloc": (c_i32, [c_p, c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_i64, c_p]),
    "bcm_restore_bwd_sync_bytes": (c_i64, [c_i64, c_i64]),
    "bcm_restore_bwd_chained": (c_i32, [c_p, c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_i32, c_i64, c_p,
                                        c_i64, c_p]),
    "bcm_restore_proj_fwd": (c_i32, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_p, c_i64, c_p, c_p]),
    "bcm_restore_proj_bwd_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i64]),
    "bcm_restore_proj_bwd": (c_i32, [c_p, c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_i64, c_p, c_p,
                                     c_p, c_i64, c_p]),
}

RESTORE_BWD_NOALLOC_MAX_TILES = 699040  # BCM_RESTORE_BWD_NOALLOC_MAX_TILES of the header

_lib = None


def lib():
    """Load (once) and return the native library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"bc_mamba_amd: native library {LIB_PATH} is not built "
                "(run `python -m bc_mamba_amd.build`); there is no CPU fallback")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.bcm_abi_version() != ABI_VERSION:
            raise RuntimeError("bc_mamba_amd: ABI version mismatch")
        _lib = handle
    return _lib


def call(name, *args):
    """Call a C-ABI entry point and turn a non-zero status into RuntimeError."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(lib().bcm_last_error().decode())


def ptr(t):
    return None if t is None else c_p(t.data_ptr())


def dtype_code(dtype):
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise RuntimeError(f"bc_mamba_amd: unsupported dtype {dtype}") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of_device(dev):
    """The current torch stream of device dev as a hipStream_t (read without
    building a torch Stream object where torch exposes the raw handle)."""
    if _raw_stream is not None:
        return c_p(_raw_stream(dev.index if dev.index is not None else torch.cuda.current_device()))
    return c_p(torch.cuda.current_stream(dev).cuda_stream)


def stream_of(t):
    """The current torch stream of t's device as a hipStream_t."""
    return stream_of_device(t.device)


def bitmask_words(L):
    return (L + 1023) // 1024 * 32


def tile_count(L):
    return (L + 63) // 64


def scan_chunking(a):
    """(pass_len, n_pass, needs_chunk_g) of the scan kernels for ScanArgs `a`
    (bcm_scan_chunking): the caller sizes chunk_g as [NC, n_pass, dstate]."""
    p, q, r = c_i32(), c_i32(), c_i32()
    call("bcm_scan_chunking", a, ctypes.byref(p), ctypes.byref(q), ctypes.byref(r))
    return p.value, q.value, bool(r.value)


SCAN_FAMILIES = {"auto": 0, "lanes": 1, "items": 2}  # enum bcm_scan_family of the header


def set_scan_family(name):
    """Process-wide depthwise scan family (bcm_set_scan_family): "auto",
    "lanes" (state lanes) or "items" (lane groups). Returns the previous
    setting's name. A forward and the backward that reads its chunk_g must
    run under the same setting."""
    prev = lib().bcm_set_scan_family(SCAN_FAMILIES[name])
    if prev < 0:
        raise RuntimeError(lib().bcm_last_error().decode())
    return {v: k for k, v in SCAN_FAMILIES.items()}[prev]


def attach_chunk_g(a, chunk_g):
    """Point ScanArgs `a` at a chunk_g buffer from the pass-state allocator
    (selective_scan_cuda.chunk_states_buffer or an equivalent that records
    the pass length it was sized for as `bcm_pass_len`)."""
    if chunk_g is None:
        a.chunk_g, a.chunk_g_bytes, a.chunk_g_pass = None, 0, 0
        return
    a.chunk_g, a.chunk_g_bytes = chunk_g.data_ptr(), chunk_g.numel() * 4
    a.chunk_g_pass = int(getattr(chunk_g, "bcm_pass_len", 0))


class HostMeta:
    """(E, max_seqlen) handed from the offsets kernel to the host through
    pinned memory. The kernel writes both values with one 64-bit store that
    goes through to memory, so the host polls the pinned words instead of
    recording an event: an event record makes the GPU write back its caches
    (several microseconds of idle device between two kernels)."""

    def __init__(self):
        self.t = torch.empty(2, dtype=torch.int32, pin_memory=True)
        self._v = self.t.numpy()

    def arm(self):
        """Call before enqueuing the offsets kernel that writes it."""
        self._v[0] = -1

    def ptr(self):
        return c_p(self.t.data_ptr())

    def wait(self, stream, timeout_s=10.0):
        """(E, max_seqlen) once written. Falls back to a sync of `stream` (a
        torch Stream, or a device whose current stream is meant), which also
        makes any pending write visible, if polling times out."""
        import time
        t0 = time.perf_counter()
        v = self._v
        while v[0] < 0:
            if time.perf_counter() - t0 > timeout_s:
                if not isinstance(stream, torch.cuda.Stream):
                    stream = torch.cuda.current_stream(stream)
                stream.synchronize()
                if v[0] < 0:
                    raise RuntimeError("bc_mamba_amd: offsets kernel did not deliver the event count")
                break
        return int(v[0]), int(v[1])
