"""One fwd+bwd pass of the event path driven straight through the C ABI,
with reusable device buffers: the kernel sequence `bench.py` times and the
full-size parity tests check.

  forward : count (bcm_extract_count_blocks: bitmask, counts, block sums)
            -> fill (bcm_extract_fill_blocks: row offsets from the block
            sums, cu_seqlens, k, u = x_conv gathered at the events, the
            tile table; E and max_seqlen written to pinned host memory,
            which the host polls while the fill runs)
            -> flat selective scan (bcm_scan_fwd)
            -> zero-order-hold restore (bcm_restore_fwd, from the bitmask
            and tile table: no t stream)
  backward: restore backward (bcm_restore_bwd_chained: one kernel, the runs
            that cross tile edges closed by look-back, where its tile grid
            fits one launch; else bcm_restore_bwd; fp32 dy)
            -> scan backward with the gather backward in the same kernel
            where the shape allows (bcm_scan_bwd_rows: du, the six
            parameter gradients and the dense dx rows)

Reference composition this replaces: e_model.py:361-409 (extraction and
gather), selective_scan_interface.py:1015-1237 (scan), e_model.py:123-161
(restore), and their autograd backward.
"""
import torch

try:
    from . import _native as nat
except ImportError:  # imported with this directory on sys.path
    import _native as nat


class FusedStep:
    """The fwd+bwd path of one workload (bc_mamba_amd.workloads.Workload).

    Event buffers are sized for the largest possible event count (every
    step of every channel), so the fill kernel can be enqueued before the
    host has read E; they are allocated once and reused by every step (a
    benchmark / serving workspace). After step(), the attributes hold the
    step's results: E, ms (max_seqlen), cu, k[:E], u[:E], tile_start,
    bitmask, y[:E] (scan out), xs (saved states), dense (restore out
    [B, L, D]), dy_restore[:E] (restore backward), du[:E], dx ([B, D, L], the
    gather backward) and grads (dA, dW_B, dW_C, ddt_idle, ddt_active, dD)."""

    KERNELS = ["count", "fill", "scan_fwd", "restore_fwd", "restore_bwd", "scan_bwd"]

    def __init__(self, w, dev, restore_bwd="auto", keep_du=True):
        """restore_bwd: "chained" (one kernel, bcm_restore_bwd_chained),
        "two_pass" (tile pass + fix-up pass, bcm_restore_bwd) or "auto": the
        chained form where its tile grid fits one launch (at most 4 blocks
        of 4 waves per CU; configs 1 and 2), else the two-pass form (the
        chained form's later launches cannot overlap the earlier ones:
        config 3, 54 against 40 us).
        keep_du=False: the step's gradient output is dx (the path's input
        gradient); where the scan backward writes dx's rows itself it then
        stores no separate du stream (dx holds the same values at the
        events), as the model's backward does. self.du is then not
        written."""
        if restore_bwd not in ("auto", "chained", "two_pass"):
            raise ValueError(f"restore_bwd must be 'auto', 'chained' or 'two_pass', not {restore_bwd!r}")
        if restore_bwd == "auto":
            waves = w.B * nat.tile_count(w.L) * -(-w.D // 64)
            cus = torch.cuda.get_device_properties(dev).multi_processor_count
            restore_bwd = "chained" if waves <= 16 * cus else "two_pass"
        self.w, self.dev, self.restore_bwd, self.keep_du = w, dev, restore_bwd, keep_du
        B, D, L = w.B, w.D, w.L
        self.NC = B * D
        i32 = dict(dtype=torch.int32, device=dev)
        self.bitmask = torch.empty((self.NC, nat.bitmask_words(L)), **i32)
        self.counts = torch.empty(self.NC, **i32)
        self.cu = torch.empty(self.NC + 1, **i32)
        self.meta_h = nat.HostMeta()
        self.bsums = torch.empty(nat.lib().bcm_extract_block_sums_bytes(self.NC) // 4, **i32)
        self.tile_start = torch.empty((self.NC, nat.tile_count(L) + 1), **i32)
        self.dense = torch.empty((B, L, D), dtype=w.dtype, device=dev)
        self.dx = torch.empty((B, D, L), dtype=w.dtype, device=dev)
        # the chained restore backward's sync area: zeroed once here, left
        # zeroed by every call
        self.sync = torch.zeros(nat.lib().bcm_restore_bwd_sync_bytes(self.NC, L) // 8, dtype=torch.int64,
                                device=dev)
        self.ws = torch.empty(nat.lib().bcm_restore_bwd_workspace_bytes(self.NC, L) // 4, dtype=torch.float32,
                              device=dev)
        cap = self.NC * L  # upper bound of E
        self.k_buf = torch.empty(cap, **i32)
        self.u_buf = torch.empty(cap, dtype=w.dtype, device=dev)
        self.y_buf = torch.empty(cap, dtype=w.dtype, device=dev)
        self.acc_buf = torch.empty(cap, dtype=torch.float32, device=dev)  # the forward's per-event state sums
        self.dy32_buf = torch.empty(cap, dtype=torch.float32, device=dev)
        self.dy_buf = self.dy32_buf if w.dtype == torch.float32 else torch.empty(cap, dtype=w.dtype, device=dev)
        self.du_buf = torch.empty(cap, dtype=w.dtype, device=dev)
        self.x = torch.empty((self.NC, max(1, -(-L // 2048)), 2 * w.N), dtype=torch.float32, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.grads = [torch.empty((w.D, w.N), **f32) for _ in range(3)] + [torch.empty(w.D, **f32) for _ in range(3)]
        self.args = self._scan_args()
        self.rows = nat.ScanRows()
        self.rows.bitmask, self.rows.mask_row_div = self.bitmask.data_ptr(), 1
        self.rows.tile_start, self.rows.seqlen, self.rows.dx = self.tile_start.data_ptr(), L, self.dx.data_ptr()
        self.E = self.ms = -1
        self.dy_out = self.dy32_buf
        self.chunk_g = self.split_ws = None
        self.events = {}

    def _scan_args(self):
        w = self.w
        a = nat.ScanArgs()
        a.n_channels, a.dim, a.dstate, a.dtype = self.NC, w.D, w.N, nat.dtype_code(w.dtype)
        a.u, a.k, a.cu_seqlens = self.u_buf.data_ptr(), self.k_buf.data_ptr(), self.cu.data_ptr()
        a.dt_idle, a.dt_active = w.dt_idle.data_ptr(), w.dt_active.data_ptr()
        a.A, a.W_B, a.W_C, a.D = w.A.data_ptr(), w.W_B.data_ptr(), w.W_C.data_ptr(), w.D_skip.data_ptr()
        a.out, a.x = self.y_buf.data_ptr(), self.x.data_ptr()
        a.acc = self.acc_buf.data_ptr()  # written by the forward, read by the backward
        a.dout, a.x_saved, a.du = self.dy_buf.data_ptr(), self.x.data_ptr(), self.du_buf.data_ptr()
        a.dA, a.dW_B, a.dW_C, a.ddt_idle, a.ddt_active, a.dD = (g.data_ptr() for g in self.grads)
        return a

    # views of the step's event-stream results
    k = property(lambda self: self.k_buf[:self.E])
    u = property(lambda self: self.u_buf[:self.E])
    y = property(lambda self: self.y_buf[:self.E])
    # the restore backward's dy as the step wrote it: fp32 (the two-pass
    # form), or u's dtype (the one-kernel form)
    dy_restore = property(lambda self: self.dy_out[:self.E])
    du = property(lambda self: self.du_buf[:self.E])

    @property
    def xs(self):
        """The saved states x [NC, n_chunks, 2N] of the step (the buffer is
        sized for the worst case; the kernels lay it out with the step's
        n_chunks = ceil(max_seqlen / 2048))."""
        nck, N2 = self.args.n_chunks, 2 * self.w.N
        return self.x.view(-1)[:self.NC * nck * N2].view(self.NC, nck, N2)

    def step(self, timed=()):
        """One fwd+bwd. Kernels named in `timed` get HIP events around them
        (on the launch stream); their (start, end) pairs collect in
        self.events."""
        w = self.w
        s = nat.stream_of(self.counts)
        P = nat.ptr
        ev = self.events

        def mark(name, fn):
            if name in timed:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                fn()
                b.record()
                ev.setdefault(name, []).append((a, b))
            else:
                fn()

        D, L = w.D, w.L
        dt = nat.dtype_code(w.dtype)
        self.meta_h.arm()
        mark("count", lambda: nat.call("bcm_extract_count_blocks", P(w.membrane), nat.dtype_code(w.membrane.dtype),
                                       self.NC, L, float(w.threshold), P(self.bitmask), P(self.counts), P(self.bsums),
                                       s))
        mark("fill", lambda: nat.call("bcm_extract_fill_blocks", P(self.bitmask), P(self.counts), P(self.bsums),
                                      self.meta_h.ptr(), self.NC, L, 1, P(w.x_conv), dt, P(self.cu), None, None,
                                      P(self.k_buf), P(self.u_buf), P(self.tile_start), s))
        E, ms = self.meta_h.wait(torch.cuda.current_stream())  # the fill keeps the GPU busy meanwhile
        if E != self.E or ms != self.ms:
            self.E, self.ms = E, ms
            a = self.args
            a.n_events, a.max_seqlen, a.n_chunks = E, ms, max(1, -(-ms // 2048))
            # pass-start states of channels longer than one pass (written by
            # the forward, read by the backward)
            pass_len, n_pass, needs = nat.scan_chunking(a)
            self.chunk_g = torch.empty((self.NC, n_pass, w.N), dtype=torch.float32, device=self.dev) \
                if needs else None
            if needs:
                self.chunk_g.bcm_pass_len = pass_len
            nat.attach_chunk_g(a, self.chunk_g)
            # parameter-gradient partials when model channels are split over workgroups
            nb = int(nat.lib().bcm_scan_bwd_workspace_bytes(a))
            self.split_ws = torch.empty(max(nb, 4) // 4, dtype=torch.float32, device=self.dev) if nb else None
            a.split_ws = self.split_ws.data_ptr() if nb else None
            a.split_ws_bytes = nb
            a.du = self.du_buf.data_ptr()
            if not self.keep_du and nat.lib().bcm_scan_bwd_rows_fused(a, self.rows) == 1:
                a.du = None
        mark("scan_fwd", lambda: nat.call("bcm_scan_fwd", self.args, s))
        mark("restore_fwd", lambda: nat.call("bcm_restore_fwd", P(self.y_buf), dt, E, P(self.bitmask), 1,
                                             P(self.tile_start), self.NC, D, L, P(self.dense), dt, s))
        if self.restore_bwd == "chained":
            # dy in the dtype the scan reads (u's): a 16-bit dy is rounded as
            # the kernel stores it, no separate cast
            self.dy_out = self.dy_buf
            mark("restore_bwd", lambda: nat.call("bcm_restore_bwd_chained", P(w.dout), dt, P(self.bitmask), 1,
                                                 P(self.tile_start), self.NC, D, L, P(self.dy_buf), dt, E,
                                                 P(self.sync), 8 * self.sync.numel(), s))
        else:
            self.dy_out = self.dy32_buf
            mark("restore_bwd", lambda: nat.call("bcm_restore_bwd", P(w.dout), dt, P(self.bitmask), 1,
                                                 P(self.tile_start), self.NC, D, L, P(self.dy32_buf), E,
                                                 P(self.ws), 4 * self.ws.numel(), s))
            if self.dy_buf is not self.dy32_buf:  # the scan takes dout in u's dtype
                self.dy_buf[:E].copy_(self.dy32_buf[:E])
        # the scan backward writes du and the dense dx rows (the gather
        # backward) in one kernel where the shape allows, else in two
        mark("scan_bwd", lambda: nat.call("bcm_scan_bwd_rows", self.args, self.rows, s))

    def kernel_ms(self, name):
        """Mean HIP-event time of the launches of `name` recorded so far."""
        torch.cuda.synchronize()
        v = [a.elapsed_time(b) for a, b in self.events.get(name, [])]
        return sum(v) / len(v) if v else float("nan")
