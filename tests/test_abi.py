"""The C-ABI library loads and exports exactly what include/bcm_event_scan.h
declares; host-side argument checks report errors without touching a GPU."""
import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (load torch's HIP runtime before the library)

import bc_mamba_amd._native as nat
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "bcm_event_scan.h")


def _header_text():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return re.sub(r"//[^\n]*", "", txt)


def header_functions():
    return set(re.findall(r"\b(bcm_[a-z0-9_]+)\s*\(", _header_text()))


def header_struct_fields(name="bcm_scan_args"):
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), _header_text(), re.S).group(1)
    return [m.group(1) for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*;", body)]


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(nat.LIB_PATH):
        from bc_mamba_amd import build
        build.build()
    return nat.lib()


def test_header_declares_exactly_the_bound_functions():
    assert header_functions() == set(nat.SIGNATURES)


def test_library_exports_every_header_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), name


def test_scan_args_layout_matches_header():
    assert [f for f, _ in nat.ScanArgs._fields_] == header_struct_fields()
    # 1 int64 + 6 int32 (= 32 bytes incl. no padding) + 27 pointers + 2 int64 sizes + int32 chunk_g_pass
    # (padded to 8 bytes for the next pointer) + the acc pointer
    assert ctypes.sizeof(nat.ScanArgs) == 8 + 6 * 4 + 27 * 8 + 2 * 8 + 8 + 8


def test_scan_bc_layout_matches_header():
    assert [f for f, _ in nat.ScanBC._fields_] == header_struct_fields("bcm_scan_bc")
    # 4 int32 + 3 int64 + 5 pointers + 2 int64
    assert ctypes.sizeof(nat.ScanBC) == 4 * 4 + 3 * 8 + 5 * 8 + 2 * 8


def test_scan_rows_layout_matches_header():
    assert [f for f, _ in nat.ScanRows._fields_] == header_struct_fields("bcm_scan_rows")
    assert ctypes.sizeof(nat.ScanRows) == 5 * 8


def test_scan_rows_arguments_are_rejected_before_launch(lib):
    a = nat.ScanArgs()
    a.n_channels, a.dim, a.dstate, a.max_seqlen, a.n_chunks, a.dtype = 4, 2, 16, 10, 1, 0
    assert lib.bcm_scan_bwd_rows(a, None, None) == 1 and "null argument" in lib.bcm_last_error().decode()
    r = nat.ScanRows()
    r.seqlen, r.mask_row_div = 64, 0
    assert lib.bcm_scan_bwd_rows(a, r, None) == 1 and "mask_row_div" in lib.bcm_last_error().decode()
    r.mask_row_div = 1
    assert lib.bcm_scan_bwd_rows(a, r, None) == 1 and "null index" in lib.bcm_last_error().decode()
    r.bitmask, r.tile_start, r.dx = 20, 16, 16  # never dereferenced: rejected first
    assert lib.bcm_scan_bwd_rows(a, r, None) == 1 and "8-byte aligned" in lib.bcm_last_error().decode()
    assert lib.bcm_scan_bwd_rows_fused(a, r) < 0 and "8-byte aligned" in lib.bcm_last_error().decode()
    # a shape the one kernel does not take (seqlen % 4 != 0): the rows come
    # from du in a second pass, so du cannot be left out
    r.bitmask, r.seqlen = 16, 63
    a.n_events, a.dout = 10, 16
    assert lib.bcm_scan_bwd_rows_fused(a, r) == 0
    assert lib.bcm_scan_bwd_rows(a, r, None) == 1 and "du required" in lib.bcm_last_error().decode()


def test_header_constants_match_binding():
    text = open(HEADER).read()
    for name, value in (("BCM_ABI_VERSION", nat.ABI_VERSION), ("BCM_SCAN_SEQLEN_EXCEEDED", nat.SCAN_SEQLEN_EXCEEDED),
                        ("BCM_SCAN_ROWS_INCOMPLETE", nat.SCAN_ROWS_INCOMPLETE),
                        ("BCM_RESTORE_BWD_NOALLOC_MAX_TILES", nat.RESTORE_BWD_NOALLOC_MAX_TILES)):
        m = re.search(r"#define\s+%s\s+(\d+)" % name, text)
        assert m and int(m.group(1)) == value, name


def test_restore_bwd_noalloc_rejects_before_launch(lib):
    """The allocation-free restore backward refuses a problem larger than
    its scratch (and invalid arguments) before touching the device."""
    L = 2048
    rows = nat.RESTORE_BWD_NOALLOC_MAX_TILES // nat.tile_count(L) + 1
    rows += (-rows) % 64  # divisible by dim
    assert lib.bcm_restore_bwd_noalloc(16, 0, 16, 1, 16, rows, 64, L, 16, 10, None) == 1
    assert "scratch limit" in lib.bcm_last_error().decode()
    assert lib.bcm_restore_bwd_noalloc(16, 9, 16, 1, 16, 64, 64, L, 16, 10, None) == 1
    assert lib.bcm_last_error().decode().startswith("bcm_restore_bwd_noalloc")


def test_restore_bwd_chained_checks_before_launch(lib):
    """The one-kernel restore backward: sync area size (two header words +
    one word per (channel, tile)) and its checks, before any launch."""
    n_rows, L = 128, 1100
    need = 8 * (2 + n_rows * nat.tile_count(L))
    assert lib.bcm_restore_bwd_sync_bytes(n_rows, L) == need
    assert lib.bcm_restore_bwd_sync_bytes(-1, L) == 0
    args = (16, 0, 16, 1, 16, n_rows, 64, L, 16, 0, 10)
    assert lib.bcm_restore_bwd_chained(*args, None, need, None) == 1
    assert "sync area of %d bytes" % need in lib.bcm_last_error().decode()
    assert lib.bcm_restore_bwd_chained(*args, 16, need - 8, None) == 1
    assert lib.bcm_restore_bwd_chained(*args, 12, need, None) == 1  # not 8-byte aligned
    assert lib.bcm_restore_bwd_chained(16, 0, 16, 1, 16, n_rows, 60, L, 16, 0, 10, 16, need, None) == 1
    assert "divisible by dim" in lib.bcm_last_error().decode()
    # dy in fp32 or dout's dtype only
    assert lib.bcm_restore_bwd_chained(16, 2, 16, 1, 16, n_rows, 64, L, 16, 1, 10, 16, need, None) == 1
    assert "dy must be fp32 or dout's dtype" in lib.bcm_last_error().decode()


def test_restore_proj_checks_before_launch(lib):
    """The fused restore -> out_proj entry points: workspace size formula
    (fix-up arrays + one d_model x dim partial per 512-step segment of each
    sequence) and argument errors raised before any launch."""
    n_rows, dim, L, dm = 128, 64, 1100, 32
    nT, n_parts = nat.tile_count(L), (n_rows // dim) * 3
    ws = lib.bcm_restore_proj_bwd_workspace_bytes(n_rows, dim, L, dm)
    assert ws == 3 * 4 * n_rows * nT + 4 * n_parts * dm * dim
    assert lib.bcm_restore_proj_bwd_workspace_bytes(n_rows, 0, L, dm) == 0
    # n_rows not a multiple of dim, d_model < 1
    assert lib.bcm_restore_proj_fwd(16, 10, 16, 1, 16, 100, 64, L, 16, None, dm, 16, None) == 1
    assert "multiple of dim" in lib.bcm_last_error().decode()
    assert lib.bcm_restore_proj_fwd(16, 10, 16, 1, 16, n_rows, dim, L, 16, None, 0, 16, None) == 1
    assert lib.bcm_last_error().decode().startswith("bcm_restore_proj_fwd")
    # workspace one byte short
    assert lib.bcm_restore_proj_bwd(16, 16, 10, 16, 1, 16, n_rows, dim, L, 16, dm, 16, 16, 16, ws - 1, None) == 1
    assert "workspace" in lib.bcm_last_error().decode()


def test_host_helpers(lib):
    assert lib.bcm_abi_version() == nat.ABI_VERSION == 4
    assert lib.bcm_bitmask_words(2048) == nat.bitmask_words(2048) == 64
    assert lib.bcm_bitmask_words(1) == 32 and lib.bcm_bitmask_words(1025) == 64
    assert lib.bcm_tile_count(2048) == nat.tile_count(2048) == 32
    assert lib.bcm_tile_count(65) == 2


def test_invalid_arguments_are_rejected_before_launch(lib):
    rc = lib.bcm_extract_count(None, 7, 4, 16, 0.5, None, None, None)
    assert rc == 1 and lib.bcm_last_error().decode().startswith("bcm_extract_count")
    assert lib.bcm_scan_fwd(None, None) == 1
    assert lib.bcm_last_error().decode().startswith("bcm_scan_fwd")
    a = nat.ScanArgs()
    a.n_channels, a.dim, a.dstate, a.max_seqlen, a.n_chunks, a.dtype = 4, 2, 300, 10, 1, 0
    assert lib.bcm_scan_bwd(a, None) == 1 and "dstate" in lib.bcm_last_error().decode()
    a.dstate, a.n_chunks = 16, 2
    assert lib.bcm_scan_fwd(a, None) == 1 and "n_chunks" in lib.bcm_last_error().decode()
    assert lib.bcm_restore_fwd(None, 0, 0, None, 1, None, 10, 3, 8, None, 0, None) == 1
    assert "divisible" in lib.bcm_last_error().decode()
    assert lib.bcm_restore_fwd(None, 1, 0, None, 1, None, 8, 4, 8, None, 0, None) == 1
    assert "fp16 input only supports fp16 output" in lib.bcm_last_error().decode()


def test_scan_var_arguments_are_rejected_before_launch(lib):
    a = nat.ScanArgs()
    a.n_channels, a.dim, a.dstate, a.max_seqlen, a.n_chunks, a.dtype = 4, 2, 16, 10, 1, 0
    a.cu_seqlens = a.dt_idle = a.dt_active = a.A = 16  # never dereferenced: rejected first
    bc = nat.ScanBC()
    bc.layout = 7
    assert lib.bcm_scan_var_fwd(a, bc, None) == 1 and "layout" in lib.bcm_last_error().decode()
    bc.layout, bc.B, bc.C = nat.BC_TILED, 16, 16
    bc.b_per_event = bc.c_per_event = 1
    assert lib.bcm_scan_var_fwd(a, bc, None) == 1 and "tile_chunk_size" in lib.bcm_last_error().decode()
    bc.layout, bc.b_row_stride, bc.c_row_stride = nat.BC_LEGACY, 0, 1
    assert lib.bcm_scan_var_fwd(a, bc, None) == 1 and "row strides" in lib.bcm_last_error().decode()
    assert lib.bcm_scan_var_workspace_bytes(1000, 16) == 64000
    assert lib.bcm_scan_var_bwd(a, None, None, 0, None) == 1
    assert lib.bcm_last_error().decode().startswith("bcm_scan_var_bwd")


def test_scan_chunk_states_size_is_checked(lib):
    """A chunk_g smaller than n_channels x n_pass x dstate floats is refused
    before any launch (the kernels would otherwise index past it)."""
    a = nat.ScanArgs()
    a.n_events, a.n_channels, a.dim, a.dstate, a.max_seqlen, a.n_chunks, a.dtype = 3000, 8, 4, 16, 1100, 1, 0
    a.cu_seqlens = a.dt_idle = a.dt_active = a.A = a.W_B = a.W_C = a.u = a.k = 16
    a.out = a.x = 16
    pass_len, n_pass, needs = nat.scan_chunking(a)
    assert needs and n_pass > 1
    a.chunk_g, a.chunk_g_bytes, a.chunk_g_pass = 16, 4 * 8 * n_pass * 16 - 4, pass_len
    assert lib.bcm_scan_fwd(a, None) == 1 and "chunk_g needs" in lib.bcm_last_error().decode()


def test_scan_refuses_chunk_states_of_another_family(lib):
    """chunk_g records the pass length it was sized for (chunk_g_pass). A
    forward run under one scan family and a backward under the other (which
    walks passes of a different length) would read the pass states at the
    wrong rows: both directions refuse a chunk_g whose pass length is not
    their own, before any launch (pointers are never dereferenced)."""
    a = nat.ScanArgs()
    a.n_events, a.n_channels, a.dim, a.dstate, a.max_seqlen, a.n_chunks, a.dtype = 8192 * 300, 8192, 256, 16, 367, 1, 0
    a.cu_seqlens = a.dt_idle = a.dt_active = a.A = a.W_B = a.W_C = a.u = a.k = 16
    a.out = a.x = 16
    a.dA = a.dW_B = a.dW_C = a.ddt_idle = a.ddt_active = a.dout = a.du = 16
    prev = nat.set_scan_family("lanes")
    try:
        lanes_pass, n_pass, needs = nat.scan_chunking(a)
        assert needs and lanes_pass == 32
        nat.set_scan_family("items")
        items_pass, items_n, _ = nat.scan_chunking(a)
        assert items_pass != lanes_pass
        # a chunk_g laid out by a forward under the state lanes, large enough
        # for either layout, refused by both directions of the lane groups
        a.chunk_g, a.chunk_g_bytes = 16, 4 * 8192 * max(n_pass, items_n) * 16
        a.chunk_g_pass = lanes_pass
        for fn in (lib.bcm_scan_fwd, lib.bcm_scan_bwd):
            assert fn(a, None) == 1
            msg = lib.bcm_last_error().decode()
            assert "passes of 32 events" in msg and f"passes of {items_pass}" in msg, msg
        # no record at all (0) is refused too
        nat.set_scan_family("lanes")
        a.chunk_g_pass = 0
        assert lib.bcm_scan_bwd(a, None) == 1 and "passes of 0 events" in lib.bcm_last_error().decode()
    finally:
        nat.set_scan_family(prev)


def test_scan_family_setter_rejects_unknown_codes(lib):
    prev = nat.set_scan_family("auto")
    try:
        assert lib.bcm_set_scan_family(7) == -1
        assert lib.bcm_last_error().decode().startswith("bcm_set_scan_family")
        assert nat.set_scan_family("items") == "auto"
        assert nat.set_scan_family("lanes") == "items"
    finally:
        nat.set_scan_family(prev)


def test_scan_backward_requires_chunk_states(lib):
    """A multi-pass backward whose passes are shorter than 2048 events needs
    the forward's pass-start states: without chunk_g it is refused before
    any launch instead of reading states it was not given (host validation
    only; the pointers are never dereferenced)."""
    a = nat.ScanArgs()
    # 16 channels, mean 150 events, one of 744: the cost model picks passes
    # much shorter than the longest channel
    a.n_events, a.n_channels, a.dim, a.dstate, a.max_seqlen, a.n_chunks, a.dtype = 2400, 16, 8, 16, 744, 1, 0
    pass_len, n_pass, needs = nat.scan_chunking(a)
    assert needs and n_pass > 1 and pass_len < 2048  # the refusal below is exercised
    a.cu_seqlens = a.dt_idle = a.dt_active = a.A = a.W_B = a.W_C = a.u = a.k = 16
    a.dA = a.dW_B = a.dW_C = a.ddt_idle = a.ddt_active = a.dout = a.du = 16
    assert lib.bcm_scan_bwd(a, None) == 1 and "chunk_g required" in lib.bcm_last_error().decode()


def test_conv_events_backward_rejects_overlapping_rows(lib):
    """dx is written with x's row strides: strides whose rows overlap (a
    broadcast batch, rows closer than L) are refused before any launch."""
    ws = 4 * 2 * 4 * 5  # B=2, D=4, L=64, K=4: pointers are never dereferenced

    def call(sb, sd):
        return lib.bcm_causal_conv1d_bwd_events(16, 0, sb, sd, 2, 4, 64, 16, None, 4, 1, 16, 10, 16, 1, 16, 16, 16,
                                                None, 16, ws, None)
    assert call(0, 64) == 1 and "overlap" in lib.bcm_last_error().decode()     # broadcast batch
    assert call(256, 32) == 1 and "overlap" in lib.bcm_last_error().decode()   # rows 32 apart, L = 64
    assert call(64, 64) == 1 and "overlap" in lib.bcm_last_error().decode()


def test_scan_family_choice_and_passes():
    """The scan family: the state lanes (32-event passes kept in chunk_g; 16
    with four states per lane) for dstate 16, 32 and 64 from 4096 channels
    on a 256-CU part (a wave of four channels per SIMD), the lane groups
    below that, other dstates always the lane groups; bcm_set_scan_family
    forces either for the process. Without a device the library assumes 256
    CUs."""
    def chunking(nc, dstate, ms):
        a = nat.ScanArgs()
        a.n_events, a.n_channels, a.dim, a.dstate, a.max_seqlen = nc * 100, nc, 256, dstate, ms
        return nat.scan_chunking(a)
    prev = nat.set_scan_family("auto")
    try:
        assert chunking(8192, 16, 367) == (32, 12, 1)      # config 1: lanes, chunk_g rows every 32 events
        assert chunking(4096, 16, 482) == (32, 16, 1)      # config 2: lanes
        assert chunking(2048, 16, 482)[0] > 32             # half the SIMDs: lane groups
        assert chunking(8192, 64, 1111) == (16, 70, 1)     # config 3: four states per lane, 16-event passes
        assert chunking(8192, 32, 367) == (32, 12, 1)      # two states per lane
        assert chunking(2048, 64, 367)[0] > 32             # half the SIMDs: lane groups
        assert chunking(8192, 48, 367)[0] > 32             # dstate 48: lane groups
        assert chunking(8192, 16, 20) == (32, 1, 0)        # one pass: no chunk_g
        nat.set_scan_family("lanes")
        assert chunking(2048, 16, 482) == (32, 16, 1)
        nat.set_scan_family("items")
        assert chunking(8192, 16, 367)[0] > 32
    finally:
        nat.set_scan_family(prev)
