"""CPU oracle of BC_mamba's event-sparse path - TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference algorithm, function by function, used
as the checker of the HIP library. Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it; the product package never does.

Integer outputs (event ids, times, gaps, offsets) are exact. Floating-point
work runs in float64 on the float32 values of the inputs, so the oracle is
at least as accurate as the fp32 reference kernels it restates.

How each function is pinned (tests/test_oracle.py):
  extract_base_events  brute force over a dense mask (np.nonzero), invariants
  expand_base_events   closed-form repeat_interleave layout, identity at 1
  gather_fwd / _bwd    closed form (the reference's own Python fallback)
  scan_fwd             independent dense formulation (oracle/torch_path.py,
                       the textbook selective_scan_ref form), closed forms for
                       one and two events, all-k=1 limit, clamp range
  scan_bwd             float64 autograd of the dense formulation, finite
                       differences, closed-form one-event gradients
  restore_fwd / _bwd   brute-force per-position loops on small inputs,
                       adjointness <restore(y), g> == <y, restore_bwd(g)>
  scan_var_fwd / _bwd  with B_i = u_i W_B and C_i = u_i W_C they reproduce the
                       depthwise scan_fwd / scan_bwd (the chain rule through
                       B and C gives du, dW_B and dW_C); finite differences
                       of every input on random per-event B and C
  bc_per_event /       brute-force loops over events for the legacy,
  bc_grad_layout       constant and tiled layouts; adjointness of the two
  pw_effective /       finite differences of the composed scan loss in pw
  pw_grads             and in W
  conv1d_fwd / _bwd    torch.nn.functional.conv1d (groups = D, padding K-1,
                       the reference's own fallback) and float64 autograd
  conv_at_events /     equal to the dense conv1d_fwd read at the events, and
  conv_bwd_events      to float64 autograd through a gather of the dense conv
  spike_ste            torch's (p >= thr).float() + p - p bit for bit, bits
                       equal to the dense s > 0.5 of the transposed spikes
"""
import math

import numpy as np

LOG2E = 1.4426950408889634
CLAMP = 126.0  # selective_scan_common.h:45 SAFE_EXP2F_RANGE
CHUNK = 2048   # selective_scan.cpp:795 n_chunks = ceil(max_seqlen / 2048)


# --------------------------------------------------------------- extraction
def extract_base_events(x, threshold):
    """extract_events_cuda.cu:324-418 (count_base_kernel :192-208 strict
    `(float)x > threshold`; fill_base_kernel :226-312 channel-major, time
    ascending, k = t+1 for a channel's first event else t - t_prev).
    x: [B, d_model, L] array (values as float32). Returns (ch, t, k, cu,
    counts, max_seqlen) with int32 arrays and a Python int."""
    B, Dm, L = x.shape
    NC = B * Dm
    mask = np.asarray(x, dtype=np.float32).reshape(NC, L) > np.float32(threshold)
    counts = mask.sum(axis=1).astype(np.int32)
    cu = np.zeros(NC + 1, dtype=np.int32)
    np.cumsum(counts, out=cu[1:])
    ch, t = np.nonzero(mask)
    ch, t = ch.astype(np.int32), t.astype(np.int32)
    first = np.ones(t.shape, dtype=bool)
    first[1:] = ch[1:] != ch[:-1]
    prev = np.empty_like(t)
    prev[1:] = t[:-1]
    k = np.where(first, t + 1, t - prev).astype(np.int32)
    return ch, t, k, cu, counts, int(counts.max()) if NC else 0


def expand_base_events(ch, t, k, cu, B, d_model, expand):
    """extract_events_cuda.cu:529-603: base channel c -> logical channels
    c*expand + r; cu_l[c*expand+r] = cu[c]*expand + r*cnt_c (:440-466);
    event i of c -> position cu[c]*expand + r*cnt_c + (i - cu[c]) (:482-509)."""
    NC = B * d_model
    cnt = np.diff(cu).astype(np.int64)
    cu_l = np.zeros(NC * expand + 1, dtype=np.int64)
    for r in range(expand):
        cu_l[np.arange(NC) * expand + r] = cu[:-1].astype(np.int64) * expand + r * cnt
    cu_l[NC * expand] = int(cu[NC]) * expand
    E = len(ch) * expand
    och, ot, ok = (np.empty(E, dtype=np.int32) for _ in range(3))
    off = np.arange(len(ch)) - cu[ch]
    for r in range(expand):
        pos = cu[ch].astype(np.int64) * expand + r * cnt[ch] + off
        och[pos] = ch * expand + r
        ot[pos] = t
        ok[pos] = k
    return och, ot, ok, cu_l.astype(np.int32), int(cnt.max()) if NC else 0


def gather_fwd(x, ch, t):
    """extract_events_cuda.cu:629-642 / e_model.py:196-201:
    out[e] = x.reshape(NC, L)[ch[e], t[e]]."""
    B, D, L = x.shape
    return np.asarray(x).reshape(B * D, L)[ch, t]


def gather_bwd(g, ch, t, NC, L):
    """extract_events_cuda.cu:649-662, :731: zeros except dx[ch, t] = g."""
    dx = np.zeros((NC, L), dtype=np.asarray(g).dtype)
    dx[ch, t] = g
    return dx


# --------------------------------------------------------------------- scan
def _padded(cu, arr, fill, dtype):
    NC = len(cu) - 1
    n = np.diff(cu)
    nmax = int(n.max()) if NC else 0
    j = np.arange(nmax)
    valid = j[None, :] < n[:, None]
    out = np.full((NC, nmax), fill, dtype=dtype)
    src = cu[:-1, None].astype(np.int64) + j[None, :]
    out[valid] = np.asarray(arr)[src[valid]]
    return out, valid, n


def _decay(delta, Al):
    """selective_scan_fwd_kernel.cuh:557-559, :650-651: exp2(clamp(Δ·A·log2e))."""
    return np.exp2(np.clip(delta * Al, -CLAMP, CLAMP))


def scan_fwd(u, k, cu, max_seqlen, dt_idle, dt_active, A, W_B, W_C, D=None, z=None):
    """Depthwise flat_ch forward (selective_scan_fwd_kernel.cuh:403-728):
      Δ_i = dt_idle[d](k_i-1) + dt_active[d]            :545
      h_i = exp2(clamp(Δ_i A log2e)) h_{i-1} + Δ_i u_i (u_i W_B)  :570-579, :651
      y_i = D u_i + Σ_s h_i (u_i W_C)                  :547, :604-611, :680-685
    x[ch, c] = (prod of a, h) after the last event of 2048-event chunk c
    (:666-677, running prefix), zeros past the channel's end (:803).
    Returns (out, x) or (out, x, out_z) with out_z = out * silu(z) (:700-716)."""
    f8 = np.float64
    NC = len(cu) - 1
    dim, N = A.shape
    d = np.arange(NC) % dim
    U, valid, n = _padded(cu, np.asarray(u, dtype=f8), 0.0, f8)
    K, _, _ = _padded(cu, k, 1, np.int64)
    nmax = U.shape[1]
    dt_i, dt_a = np.asarray(dt_idle, f8)[d], np.asarray(dt_active, f8)[d]
    delta = dt_i[:, None] * (K - 1) + dt_a[:, None]
    Al = np.asarray(A, f8)[d] * LOG2E
    WB, WC = np.asarray(W_B, f8)[d], np.asarray(W_C, f8)[d]
    Dv = np.asarray(D, f8)[d] if D is not None else np.zeros(NC)
    n_chunks = max(1, math.ceil(int(max_seqlen) / CHUNK))
    x = np.zeros((NC, n_chunks, 2 * N))
    h = np.zeros((NC, N))
    P = np.ones((NC, N))
    Y = np.zeros((NC, nmax))
    for i in range(nmax):
        v = valid[:, i]
        a = _decay(delta[:, i, None], Al)
        hn = a * h + delta[:, i, None] * U[:, i, None] ** 2 * WB
        h = np.where(v[:, None], hn, h)
        P = np.where(v[:, None], P * a, P)
        Y[:, i] = Dv * U[:, i] + U[:, i] * (h * WC).sum(axis=1)
        c = i // CHUNK
        at_end = v & (((i + 1) % CHUNK == 0) | (i + 1 == n))
        rows = np.nonzero(at_end & (c < n_chunks))[0]
        x[rows, c, 0::2] = P[rows]
        x[rows, c, 1::2] = h[rows]
    out = Y[valid]
    if z is None:
        return out, x
    zf = np.asarray(z, f8)
    return out, x, out * (zf / (1.0 + np.exp(-zf)))


def scan_bwd(u, k, cu, max_seqlen, dt_idle, dt_active, A, W_B, W_C, dout, D=None, z=None, out=None):
    """Depthwise flat_ch backward (selective_scan_bwd_kernel.cuh:761-1168):
      z gate  dz = dout·out·σ(z)(1 + z(1-σ(z))), dout <- dout·silu(z)     :795-801
      dx_i    = dout_i u_i W_C + a_{i+1} dx_{i+1}                            :902-935
      du_i    = D dout_i + Σ_s [2 dx Δ u W_B + dout h W_C]                   :816-818, :944-995
      dΔ_i    = Σ_s [dx u² W_B + dx A a_i h_{i-1}]                           :946-947
      dA     += dx Δ a_i h_{i-1};  dW_B += dx Δ u²;  dW_C += dout h u       :948, :983-1004
      dD     += dout u;  ddt_idle += dΔ (k-1);  ddt_active += dΔ           :820, :1064-1068
    The Δ-derivative of the decay is A·a even where the exponent is clamped,
    as in the reference. Parameter gradients are summed over all channels
    with d = ch % dim. Returns (du, dA, dW_B, dW_C, ddt_idle, ddt_active,
    dD or None, dz or None)."""
    f8 = np.float64
    NC = len(cu) - 1
    dim, N = A.shape
    d = np.arange(NC) % dim
    U, valid, n = _padded(cu, np.asarray(u, f8), 0.0, f8)
    K, _, _ = _padded(cu, k, 1, np.int64)
    DO, _, _ = _padded(cu, np.asarray(dout, f8), 0.0, f8)
    dz = None
    if z is not None:
        Z, _, _ = _padded(cu, np.asarray(z, f8), 0.0, f8)
        O, _, _ = _padded(cu, np.asarray(out, f8), 0.0, f8)
        sg = 1.0 / (1.0 + np.exp(-Z))
        dzp = DO * O * sg * (1.0 + Z * (1.0 - sg))
        dz = dzp[valid]
        DO = DO * Z * sg
    nmax = U.shape[1]
    dt_i, dt_a = np.asarray(dt_idle, f8)[d], np.asarray(dt_active, f8)[d]
    delta = dt_i[:, None] * (K - 1) + dt_a[:, None]
    Araw = np.asarray(A, f8)[d]
    Al = Araw * LOG2E
    WB, WC = np.asarray(W_B, f8)[d], np.asarray(W_C, f8)[d]
    Dv = np.asarray(D, f8)[d] if D is not None else np.zeros(NC)
    # forward states
    a_all = np.ones((NC, nmax, N))
    h_all = np.zeros((NC, nmax, N))
    h = np.zeros((NC, N))
    for i in range(nmax):
        v = valid[:, i, None]
        a = _decay(delta[:, i, None], Al)
        hn = a * h + delta[:, i, None] * U[:, i, None] ** 2 * WB
        a_all[:, i] = np.where(v, a, 1.0)
        h = np.where(v, hn, h)
        h_all[:, i] = h
    du = np.zeros((NC, nmax))
    ddelta = np.zeros((NC, nmax))
    dA_c, dWB_c, dWC_c = np.zeros((NC, N)), np.zeros((NC, N)), np.zeros((NC, N))
    dx = np.zeros((NC, N))
    for i in range(nmax - 1, -1, -1):
        v = valid[:, i, None]
        a_next = a_all[:, i + 1] if i + 1 < nmax else np.ones((NC, N))
        dx = np.where(v, DO[:, i, None] * U[:, i, None] * WC + a_next * dx, 0.0)
        hprev = h_all[:, i - 1] if i > 0 else np.zeros((NC, N))
        ah = a_all[:, i] * hprev
        hi = h_all[:, i]
        du[:, i] = Dv * DO[:, i] + (2.0 * delta[:, i, None] * U[:, i, None] * dx * WB).sum(1) \
            + DO[:, i] * (hi * WC).sum(1)
        ddelta[:, i] = (dx * U[:, i, None] ** 2 * WB).sum(1) + (dx * Araw * ah).sum(1)
        dA_c += dx * delta[:, i, None] * ah
        dWB_c += dx * delta[:, i, None] * U[:, i, None] ** 2
        dWC_c += np.where(v, DO[:, i, None] * U[:, i, None] * hi, 0.0)
    ddelta = np.where(valid, ddelta, 0.0)
    dD_c = (DO * U).sum(1)
    ddti_c = (ddelta * (K - 1)).sum(1)
    ddta_c = ddelta.sum(1)

    def per_dim(v):
        outv = np.zeros((dim,) + v.shape[1:])
        np.add.at(outv, d, v)
        return outv

    return (du[valid], per_dim(dA_c), per_dim(dWB_c), per_dim(dWC_c), per_dim(ddti_c), per_dim(ddta_c),
            per_dim(dD_c) if D is not None else None, dz)


# ------------------------------------------- scan with per-event B and C
def bc_per_event(Bt, cu, dim, N, tile_offsets=None, tile_chunk_size=0):
    """Per-event values [E, N] of a non-depthwise B or C operand of
    fwd_flat_ch / bwd_flat_ch (selective_scan.cpp:768-776, 840-848):
      legacy [N, E]    B[s, e]                       (selective_scan_fwd_kernel.cuh:588-591)
      constant [N, dim] B[s, ch % dim] for every event (:592-598, bwd only)
      tiled [NT, N, T]  B[tile_offsets[ch] + p // T, s, p % T] for the
                        event at position p of channel ch (:580-587)."""
    Bt = np.asarray(Bt, np.float64)
    cu = np.asarray(cu, np.int64)
    NC = len(cu) - 1
    E = int(cu[-1])
    ch = np.repeat(np.arange(NC), np.diff(cu))
    if tile_offsets is not None:
        T = int(tile_chunk_size)
        p = np.arange(E) - cu[ch]
        tiles = np.asarray(tile_offsets, np.int64)[ch] + p // T
        return Bt[tiles, :, p % T]
    if Bt.shape[1] == E:
        return Bt.T.copy()
    assert Bt.shape[1] == dim
    return Bt[:, ch % dim].T.copy()


def bc_grad_layout(dev, like_shape, cu, dim, tile_offsets=None, tile_chunk_size=0):
    """Inverse of bc_per_event for gradients: per-event [E, N] values into
    the operand's layout (legacy: transpose; constant: summed over the events
    of each d; tiled: scattered, zeros where no event maps)."""
    cu = np.asarray(cu, np.int64)
    NC = len(cu) - 1
    E = int(cu[-1])
    ch = np.repeat(np.arange(NC), np.diff(cu))
    if tile_offsets is not None:
        T = int(tile_chunk_size)
        p = np.arange(E) - cu[ch]
        tiles = np.asarray(tile_offsets, np.int64)[ch] + p // T
        out = np.zeros(like_shape)
        out[tiles, :, p % T] = dev
        return out
    if like_shape[1] == E:
        return dev.T.copy()
    out = np.zeros(like_shape)
    np.add.at(out.T, ch % dim, dev)
    return out


def scan_var_fwd(u, k, cu, max_seqlen, dt_idle, dt_active, A, Bev, Cev, D=None, z=None):
    """flat_ch forward with per-event B and C (selective_scan_fwd_kernel.cuh
    :566-686, the variable-B/C branch):
      h_i = exp2(clamp(Δ_i A log2e)) h_{i-1} + B_i Δ_i u_i      :650-652
      y_i = D u_i + Σ_s C_i h_i                                 :680-685
    Bev, Cev: [E, N] per-event values (bc_per_event). x as in scan_fwd."""
    f8 = np.float64
    NC = len(cu) - 1
    dim, N = A.shape
    d = np.arange(NC) % dim
    U, valid, n = _padded(cu, np.asarray(u, dtype=f8), 0.0, f8)
    K, _, _ = _padded(cu, k, 1, np.int64)
    nmax = U.shape[1]
    Bp = np.zeros((NC, nmax, N))
    Cp = np.zeros((NC, nmax, N))
    src = np.asarray(cu[:-1], np.int64)[:, None] + np.arange(nmax)[None, :]
    Bp[valid] = np.asarray(Bev, f8)[src[valid]]
    Cp[valid] = np.asarray(Cev, f8)[src[valid]]
    dt_i, dt_a = np.asarray(dt_idle, f8)[d], np.asarray(dt_active, f8)[d]
    delta = dt_i[:, None] * (K - 1) + dt_a[:, None]
    Al = np.asarray(A, f8)[d] * LOG2E
    Dv = np.asarray(D, f8)[d] if D is not None else np.zeros(NC)
    n_chunks = max(1, math.ceil(int(max_seqlen) / CHUNK))
    x = np.zeros((NC, n_chunks, 2 * N))
    h = np.zeros((NC, N))
    P = np.ones((NC, N))
    Y = np.zeros((NC, nmax))
    for i in range(nmax):
        v = valid[:, i]
        a = _decay(delta[:, i, None], Al)
        hn = a * h + Bp[:, i] * (delta[:, i] * U[:, i])[:, None]
        h = np.where(v[:, None], hn, h)
        P = np.where(v[:, None], P * a, P)
        Y[:, i] = Dv * U[:, i] + (Cp[:, i] * h).sum(axis=1)
        c = i // CHUNK
        at_end = v & (((i + 1) % CHUNK == 0) | (i + 1 == n))
        rows = np.nonzero(at_end & (c < n_chunks))[0]
        x[rows, c, 0::2] = P[rows]
        x[rows, c, 1::2] = h[rows]
    out = Y[valid]
    if z is None:
        return out, x
    zf = np.asarray(z, f8)
    return out, x, out * (zf / (1.0 + np.exp(-zf)))


def scan_var_bwd(u, k, cu, max_seqlen, dt_idle, dt_active, A, Bev, Cev, dout, D=None, z=None, out=None):
    """flat_ch backward with per-event B and C (selective_scan_bwd_kernel.cuh
    :902-1044, the variable-B/C branch):
      dh_i  = C_i dout_i + a_{i+1} dh_{i+1}
      dC_i  = dout_i h_i;   dB_i = dh_i Δ_i u_i
      du_i  = D dout_i + Σ_s dh_i B_i Δ_i
      dΔ_i  = Σ_s [dh_i B_i u_i + dh_i A a_i h_{i-1}]
      dA   += dh_i Δ_i a_i h_{i-1};  dD, ddt_* and the z gate as scan_bwd.
    Returns (du, dA, dBev [E, N], dCev [E, N], ddt_idle, ddt_active,
    dD or None, dz or None)."""
    f8 = np.float64
    NC = len(cu) - 1
    dim, N = A.shape
    d = np.arange(NC) % dim
    U, valid, n = _padded(cu, np.asarray(u, f8), 0.0, f8)
    K, _, _ = _padded(cu, k, 1, np.int64)
    DO, _, _ = _padded(cu, np.asarray(dout, f8), 0.0, f8)
    nmax = U.shape[1]
    Bp = np.zeros((NC, nmax, N))
    Cp = np.zeros((NC, nmax, N))
    src = np.asarray(cu[:-1], np.int64)[:, None] + np.arange(nmax)[None, :]
    Bp[valid] = np.asarray(Bev, f8)[src[valid]]
    Cp[valid] = np.asarray(Cev, f8)[src[valid]]
    dz = None
    if z is not None:
        Z, _, _ = _padded(cu, np.asarray(z, f8), 0.0, f8)
        O, _, _ = _padded(cu, np.asarray(out, f8), 0.0, f8)
        sg = 1.0 / (1.0 + np.exp(-Z))
        dz = (DO * O * sg * (1.0 + Z * (1.0 - sg)))[valid]
        DO = DO * Z * sg
    dt_i, dt_a = np.asarray(dt_idle, f8)[d], np.asarray(dt_active, f8)[d]
    delta = dt_i[:, None] * (K - 1) + dt_a[:, None]
    Araw = np.asarray(A, f8)[d]
    Al = Araw * LOG2E
    Dv = np.asarray(D, f8)[d] if D is not None else np.zeros(NC)
    a_all = np.ones((NC, nmax, N))
    h_all = np.zeros((NC, nmax, N))
    h = np.zeros((NC, N))
    for i in range(nmax):
        v = valid[:, i, None]
        a = _decay(delta[:, i, None], Al)
        hn = a * h + Bp[:, i] * (delta[:, i] * U[:, i])[:, None]
        a_all[:, i] = np.where(v, a, 1.0)
        h = np.where(v, hn, h)
        h_all[:, i] = h
    du = np.zeros((NC, nmax))
    ddelta = np.zeros((NC, nmax))
    dBp, dCp = np.zeros((NC, nmax, N)), np.zeros((NC, nmax, N))
    dA_c = np.zeros((NC, N))
    dh = np.zeros((NC, N))
    for i in range(nmax - 1, -1, -1):
        v = valid[:, i, None]
        a_next = a_all[:, i + 1] if i + 1 < nmax else np.ones((NC, N))
        dh = np.where(v, Cp[:, i] * DO[:, i, None] + a_next * dh, 0.0)
        hprev = h_all[:, i - 1] if i > 0 else np.zeros((NC, N))
        ah = a_all[:, i] * hprev
        du[:, i] = Dv * DO[:, i] + (dh * Bp[:, i]).sum(1) * delta[:, i]
        ddelta[:, i] = (dh * Bp[:, i]).sum(1) * U[:, i] + (dh * Araw * ah).sum(1)
        dA_c += dh * delta[:, i, None] * ah
        dBp[:, i] = dh * (delta[:, i] * U[:, i])[:, None]
        dCp[:, i] = np.where(v, DO[:, i, None] * h_all[:, i], 0.0)
    ddelta = np.where(valid, ddelta, 0.0)
    dD_c = (DO * U).sum(1)
    ddti_c = (ddelta * (K - 1)).sum(1)
    ddta_c = ddelta.sum(1)

    def per_dim(v):
        outv = np.zeros((dim,) + v.shape[1:])
        np.add.at(outv, d, v)
        return outv

    return (du[valid], per_dim(dA_c), dBp[valid], dCp[valid], per_dim(ddti_c), per_dim(ddta_c),
            per_dim(dD_c) if D is not None else None, dz)


def pw_effective(pw, W):
    """Depthwise + pointwise mode (selective_scan_fwd_kernel.cuh:486-509):
    W_eff[d, s] = Σ_{d'} pw[d, d'] W[d', s]."""
    return np.asarray(pw, np.float64) @ np.asarray(W, np.float64)


def pw_grads(pw, W, dW_eff):
    """Chain rule of pw_effective (selective_scan_bwd_kernel.cuh:1122-1166):
    dW[d', s] = Σ_d pw[d, d'] dW_eff[d, s],  dpw[d, d'] = Σ_s dW_eff[d, s] W[d', s]."""
    pw, W, g = (np.asarray(v, np.float64) for v in (pw, W, dW_eff))
    return pw.T @ g, g @ W.T


# ------------------------------------------------- causal conv1d + SiLU
def conv1d_fwd(x, w, bias=None, silu=True):
    """e_model.py:442-451: out[b,d,t] = act(bias[d] + Σ_k w[d,k] x[b,d,t-(K-1)+k]),
    x = 0 before t = 0, act = SiLU or identity. x [B, D, L], w [D, K]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    B, D, L = x.shape
    K = w.shape[1]
    xp = np.concatenate([np.zeros((B, D, K - 1)), x], axis=2)
    pre = np.zeros((B, D, L)) + (np.asarray(bias, np.float64)[None, :, None] if bias is not None else 0.0)
    for k in range(K):
        pre += w[None, :, k, None] * xp[:, :, k:k + L]
    return pre / (1.0 + np.exp(-pre)) if silu else pre


def conv1d_bwd(x, w, bias, dout, silu=True):
    """Gradients of conv1d_fwd: (dx, dw [D, K], dbias [D])."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    B, D, L = x.shape
    K = w.shape[1]
    pre = conv1d_fwd(x, w, bias, silu=False)
    g = np.asarray(dout, np.float64)
    if silu:
        sg = 1.0 / (1.0 + np.exp(-pre))
        g = g * sg * (1.0 + pre * (1.0 - sg))
    xp = np.concatenate([np.zeros((B, D, K - 1)), x], axis=2)
    gp = np.concatenate([g, np.zeros((B, D, K - 1))], axis=2)
    dx = np.zeros((B, D, L))
    dw = np.zeros((D, K))
    for k in range(K):
        dx += w[None, :, k, None] * gp[:, :, K - 1 - k:K - 1 - k + L]
        dw[:, k] = (g * xp[:, :, k:k + L]).sum(axis=(0, 2))
    return dx, dw, g.sum(axis=(0, 2))


def conv_at_events(x, w, bias, ch, t, silu=True):
    """The conv + SiLU evaluated only at the events (ch, t) of the flat
    channels x [NC, L] (channel ch uses w[ch % D]): x_events[e] =
    act(bias + Σ_k w[k] x[ch, t-(K-1)+k]), e_model.py:442-451 followed by
    the gather of :403-406."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    D, K = w.shape
    ch = np.asarray(ch, np.int64)
    t = np.asarray(t, np.int64)
    d = ch % D
    pre = np.asarray(bias, np.float64)[d] if bias is not None else np.zeros(len(ch))
    for k in range(K):
        tt = t - (K - 1) + k
        pre = pre + w[d, k] * np.where(tt >= 0, x[ch, np.maximum(tt, 0)], 0.0)
    return pre / (1.0 + np.exp(-pre)) if silu else pre


def conv_bwd_events(x, w, bias, du, ch, t, silu=True):
    """Backward of conv_at_events from du [E]: the gather backward (du at
    the events, 0 elsewhere) followed by conv1d_bwd over the rows of x
    [B, D, L]. Returns (dx [B, D, L], dw [D, K], dbias [D])."""
    x = np.asarray(x, np.float64)
    B, D, L = x.shape
    dense = gather_bwd(np.asarray(du, np.float64), ch, t, B * D, L).reshape(B, D, L)
    return conv1d_bwd(x, w, bias, dense, silu)


# -------------------------------------------------------------- spike head
def spike_ste(p, threshold):
    """SpikeSamplerSurrogate mode "ste" (e_model.py:233-254) on p [B, L, Dm]:
    (s, bits) with s = (p >= thr) + p - p evaluated left to right in
    float32 (the reference's dtype), and bits [B*Dm, L] bool the spikes of
    the transposed rows (b, d), the membrane the next block extracts."""
    p = np.asarray(p, np.float32)
    thr = np.float32(threshold)
    hard = (p >= thr).astype(np.float32)
    s = (hard + p) - p
    B, L, Dm = p.shape
    return s, (p >= thr).transpose(0, 2, 1).reshape(B * Dm, L)


# ------------------------------------------------------------------ restore
def restore_fwd(y, t, cu, dim, L):
    """restore_dense_fwd_kernel.cuh:38-114: out[b, t, d] = y[e] for the last
    event e of channel b*dim+d with t_e <= t (upper_bound search, :93-99),
    0 before the first event. Returns float64 (B, L, dim)."""
    NC = len(cu) - 1
    out = np.zeros((NC // dim, L, dim))
    pos = np.arange(L)
    y = np.asarray(y, dtype=np.float64)
    for c in range(NC):
        s, e = int(cu[c]), int(cu[c + 1])
        if e == s:
            continue
        j = np.searchsorted(t[s:e], pos, side="right") - 1
        out[c // dim, :, c % dim] = np.where(j >= 0, y[s + np.maximum(j, 0)], 0.0)
    return out


def restore_bwd(dout, t, cu, dim, L):
    """restore_dense_bwd_kernel.cuh:42-112: dy[e] = Σ dout[b, t, d] over the
    positions t whose last event at or before t is e. Returns float64 [E]."""
    NC = len(cu) - 1
    dy = np.zeros(int(cu[NC]))
    pos = np.arange(L)
    g_all = np.asarray(dout, dtype=np.float64)
    for c in range(NC):
        s, e = int(cu[c]), int(cu[c + 1])
        if e == s:
            continue
        j = np.searchsorted(t[s:e], pos, side="right") - 1
        keep = j >= 0
        dy[s:e] += np.bincount(j[keep], weights=g_all[c // dim, keep, c % dim], minlength=e - s)
    return dy
