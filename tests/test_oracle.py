"""Pins the CPU oracle (oracle/event_path.py) against independent
formulations, closed forms, brute force and invariants. No GPU needed."""
import math

import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import event_path as orc
from oracle import torch_path as tp

RNG = np.random.default_rng(1234)


def _params(D, N, rng):
    f32 = np.float32
    dt_i = np.log1p(np.exp(rng.standard_normal(D) - 2.0)).astype(f32)
    dt_a = np.log1p(np.exp(rng.standard_normal(D) - 2.0)).astype(f32)
    A = (-np.exp(rng.random((D, N)) * math.log(16.0))).astype(f32)
    WB = (rng.standard_normal((D, N)) / math.sqrt(N)).astype(f32)
    WC = (rng.standard_normal((D, N)) / math.sqrt(N)).astype(f32)
    Dv = rng.standard_normal(D).astype(f32)
    return dt_i, dt_a, A, WB, WC, Dv


def _stream(B, D, L, p, rng):
    mem = (rng.random((B, D, L)) < p).astype(np.float32)
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem, 0.5)
    return mem, ch, t, k, cu, ms


# ------------------------------------------------------------- extraction
def test_extract_brute_force():
    x = RNG.standard_normal((2, 3, 37)).astype(np.float32)
    ch, t, k, cu, counts, ms = orc.extract_base_events(x, 0.25)
    exp_ch, exp_t, exp_k = [], [], []
    for c in range(6):
        prev = -1
        for s in range(37):
            if x.reshape(6, 37)[c, s] > np.float32(0.25):
                exp_ch.append(c)
                exp_t.append(s)
                exp_k.append(s + 1 if prev < 0 else s - prev)
                prev = s
    assert ch.tolist() == exp_ch and t.tolist() == exp_t and k.tolist() == exp_k
    assert cu[0] == 0 and cu[-1] == len(exp_t)
    assert ms == max(np.bincount(np.array(exp_ch), minlength=6))


def test_extract_strict_threshold_and_invariants():
    x = np.array([[[0.5, 0.5000001, 0.4999, 1.0, 0.5]]], dtype=np.float32)
    ch, t, k, cu, counts, ms = orc.extract_base_events(x, 0.5)
    assert t.tolist() == [1, 3] and k.tolist() == [2, 2]
    mem, ch, t, k, cu, ms = _stream(3, 5, 200, 0.2, RNG)
    assert np.all(np.diff(cu) >= 0) and np.all(np.diff(ch) >= 0)
    for c in range(15):
        s, e = cu[c], cu[c + 1]
        assert np.array_equal(np.cumsum(k[s:e]) - 1, t[s:e])  # gaps rebuild the times
        assert np.all(ch[s:e] == c)


def test_expand_closed_form():
    mem, ch, t, k, cu, ms = _stream(2, 3, 50, 0.3, RNG)
    e1 = orc.expand_base_events(ch, t, k, cu, 2, 3, 1)
    assert all(np.array_equal(a, b) for a, b in zip(e1[:4], (ch, t, k, cu)))
    och, ot, ok, ocu, oms = orc.expand_base_events(ch, t, k, cu, 2, 3, 3)
    # logical channel c*3+r holds exactly the events of base channel c
    for c in range(6):
        for r in range(3):
            lc = c * 3 + r
            s, e = ocu[lc], ocu[lc + 1]
            assert np.all(och[s:e] == lc)
            assert np.array_equal(ot[s:e], t[cu[c]:cu[c + 1]])
            assert np.array_equal(ok[s:e], k[cu[c]:cu[c + 1]])
    assert oms == ms


def test_gather_roundtrip():
    x = RNG.standard_normal((2, 3, 40)).astype(np.float32)
    mem, ch, t, k, cu, ms = _stream(2, 3, 40, 0.3, RNG)
    u = orc.gather_fwd(x, ch, t)
    dx = orc.gather_bwd(u, ch, t, 6, 40)
    assert np.array_equal(dx[mem.reshape(6, 40) > 0.5], x.reshape(6, 40)[mem.reshape(6, 40) > 0.5])
    assert np.all(dx[mem.reshape(6, 40) <= 0.5] == 0)


# ------------------------------------------------------------------- scan
def test_scan_one_event_closed_form():
    dt_i, dt_a, A, WB, WC, Dv = _params(1, 4, RNG)
    u = np.array([0.7], np.float32)
    k = np.array([5], np.int32)
    cu = np.array([0, 1], np.int32)
    out, x = orc.scan_fwd(u, k, cu, 1, dt_i, dt_a, A, WB, WC, Dv)
    delta = float(dt_i[0]) * 4 + float(dt_a[0])
    uu = float(u[0])
    want = float(Dv[0]) * uu + delta * uu ** 3 * float(np.dot(WB[0].astype(np.float64), WC[0]))
    assert out[0] == pytest.approx(want, rel=1e-12)
    assert np.allclose(x[0, 0, 1::2], delta * uu * uu * WB[0].astype(np.float64))
    assert np.allclose(x[0, 0, 0::2], np.exp(delta * A[0].astype(np.float64)))


def test_scan_two_events_closed_form():
    dt_i, dt_a, A, WB, WC, Dv = _params(1, 3, RNG)
    u = np.array([0.4, -1.3], np.float32)
    k = np.array([1, 3], np.int32)
    cu = np.array([0, 2], np.int32)
    out, x = orc.scan_fwd(u, k, cu, 2, dt_i, dt_a, A, WB, WC, Dv)
    f = lambda v: np.asarray(v, np.float64)
    d1, d2 = f(dt_a[0]), f(dt_i[0]) * 2 + f(dt_a[0])
    h1 = d1 * f(u[0]) ** 2 * f(WB[0])
    h2 = np.exp(d2 * f(A[0])) * h1 + d2 * f(u[1]) ** 2 * f(WB[0])
    assert out[1] == pytest.approx(f(Dv[0]) * f(u[1]) + f(u[1]) * np.dot(h2, f(WC[0])), rel=1e-12)
    assert np.allclose(x[0, 0, 1::2], h2)


@pytest.mark.parametrize("clamp_regime", [False, True])
def test_scan_fwd_matches_dense_formulation(clamp_regime):
    B, D, L, N = 2, 6, 90, 5
    mem, ch, t, k, cu, ms = _stream(B, D, L, 0.25, RNG)
    dt_i, dt_a, A, WB, WC, Dv = _params(D, N, RNG)
    if clamp_regime:  # long gaps with large |A| exercise the exp2 clamp
        A = (A * 800.0).astype(np.float32)
    u = RNG.standard_normal(len(ch)).astype(np.float32)
    out, x = orc.scan_fwd(u, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv)
    T = lambda a: torch.from_numpy(np.asarray(a))
    ref = tp.scan_dense(T(u), T(k).long(), T(ch).long(), T(cu).long(), T(dt_i), T(dt_a), T(A), T(WB), T(WC),
                        T(Dv), dtype=torch.float64)
    assert_close(out, ref.numpy(), rtol=1e-12, atol_rel=1e-13, name="scan_fwd vs dense")


def test_scan_fwd_all_k1_is_dense_mamba_with_constant_delta():
    # every step an event: the flat scan is the dense recurrence with Δ = dt_active
    D, L, N = 3, 25, 4
    dt_i, dt_a, A, WB, WC, Dv = _params(D, N, RNG)
    u = RNG.standard_normal((1, D, L)).astype(np.float32)
    ch = np.repeat(np.arange(D), L).astype(np.int32)
    k = np.ones(D * L, np.int32)
    cu = (np.arange(D + 1) * L).astype(np.int32)
    out, x = orc.scan_fwd(u.reshape(-1), k, cu, L, dt_i, dt_a, A, WB, WC, Dv)
    for d in range(D):
        h = np.zeros(N)
        for s in range(L):
            ud = float(u[0, d, s])
            wb, wc = WB[d].astype(np.float64), WC[d].astype(np.float64)
            h = np.exp(float(dt_a[d]) * A[d].astype(np.float64)) * h + float(dt_a[d]) * ud * ud * wb
            assert out[d * L + s] == pytest.approx(float(Dv[d]) * ud + ud * float(h @ wc), rel=1e-10)


def test_scan_chunk_state_semantics():
    # a channel of 2500 events: x[:,0] is the state after event 2047, x[:,1] after the last
    N = 3
    dt_i, dt_a, A, WB, WC, Dv = _params(1, N, RNG)
    n = 2500
    u = RNG.standard_normal(n).astype(np.float32) * 0.3
    k = RNG.integers(1, 4, n).astype(np.int32)
    cu = np.array([0, n], np.int32)
    _, x = orc.scan_fwd(u, k, cu, n, dt_i, dt_a, A * 0.01, WB, WC, Dv)
    _, x_head = orc.scan_fwd(u[:2048], k[:2048], np.array([0, 2048], np.int32), 2048, dt_i, dt_a, A * 0.01, WB,
                             WC, Dv)
    assert x.shape == (1, 2, 2 * N)
    assert np.allclose(x[0, 0], x_head[0, 0], rtol=1e-12)
    _, x_all = orc.scan_fwd(u, k, cu, 4096 + 1, dt_i, dt_a, A * 0.01, WB, WC, Dv)
    assert x_all.shape == (1, 3, 2 * N) and np.all(x_all[0, 2] == 0)


def _bwd_case(B, D, L, N, p, with_z, rng):
    mem, ch, t, k, cu, ms = _stream(B, D, L, p, rng)
    dt_i, dt_a, A, WB, WC, Dv = _params(D, N, rng)
    E = len(ch)
    u = rng.standard_normal(E).astype(np.float32)
    dout = rng.standard_normal(E).astype(np.float32)
    z = rng.standard_normal(E).astype(np.float32) if with_z else None
    return ch, t, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv, u, dout, z


@pytest.mark.parametrize("with_z", [False, True])
def test_scan_bwd_matches_float64_autograd(with_z):
    ch, t, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv, u, dout, z = _bwd_case(2, 4, 60, 5, 0.3, with_z, RNG)
    out, x, *rest = orc.scan_fwd(u, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv, z)
    got = orc.scan_bwd(u, k, cu, ms, dt_i, dt_a, A, WB, WC, dout, Dv, z, out if with_z else None)
    T = lambda a: torch.tensor(np.asarray(a), dtype=torch.float64)
    leaves = [T(v).requires_grad_(True) for v in (u, dt_i, dt_a, A, WB, WC, Dv)]
    uu, dti, dta, A_, WB_, WC_, D_ = leaves
    y = tp.scan_dense(uu, torch.from_numpy(k).long(), torch.from_numpy(ch).long(), torch.from_numpy(cu).long(),
                      dti, dta, A_, WB_, WC_, D_, dtype=torch.float64)
    if with_z:
        zt = T(z).requires_grad_(True)
        y = y * torch.nn.functional.silu(zt)
        leaves.append(zt)
    y.backward(T(dout))
    du, dA, dWB, dWC, ddti, ddta, dD, dz = got
    for name, mine, ref in [("du", du, uu.grad), ("dA", dA, A_.grad), ("dW_B", dWB, WB_.grad),
                            ("dW_C", dWC, WC_.grad), ("ddt_idle", ddti, dti.grad), ("ddt_active", ddta, dta.grad),
                            ("dD", dD, D_.grad)] + ([("dz", dz, leaves[-1].grad)] if with_z else []):
        assert_close(mine, ref.numpy(), rtol=1e-10, atol_rel=1e-12, name=name)


def test_scan_bwd_finite_difference():
    ch, t, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv, u, dout, _ = _bwd_case(1, 2, 30, 3, 0.4, False, RNG)
    du, dA, *_ = orc.scan_bwd(u, k, cu, ms, dt_i, dt_a, A, WB, WC, dout, Dv)
    f8 = lambda v: np.asarray(v, np.float64)
    loss = lambda uu, AA: float(np.dot(orc.scan_fwd(uu, k, cu, ms, dt_i, dt_a, AA, WB, WC, Dv)[0], f8(dout)))
    eps = 1e-6
    for i in (0, len(u) // 2, len(u) - 1):
        up, um = f8(u).copy(), f8(u).copy()
        up[i] += eps
        um[i] -= eps
        assert (loss(up, f8(A)) - loss(um, f8(A))) / (2 * eps) == pytest.approx(du[i], rel=1e-6, abs=1e-9)
    Ap, Am = f8(A).copy(), f8(A).copy()
    Ap[1, 2] += eps
    Am[1, 2] -= eps
    assert (loss(f8(u), Ap) - loss(f8(u), Am)) / (2 * eps) == pytest.approx(dA[1, 2], rel=1e-6, abs=1e-9)


def test_scan_bwd_one_event_closed_form():
    dt_i, dt_a, A, WB, WC, Dv = _params(1, 4, RNG)
    u = np.array([0.9], np.float32)
    k = np.array([3], np.int32)
    cu = np.array([0, 1], np.int32)
    g = np.array([1.0], np.float32)
    du, dA, dWB, dWC, ddti, ddta, dD, _ = orc.scan_bwd(u, k, cu, 1, dt_i, dt_a, A, WB, WC, g, Dv)
    f = lambda v: np.asarray(v, np.float64)
    delta = f(dt_i[0]) * 2 + f(dt_a[0])
    s = float(np.dot(f(WB[0]), f(WC[0])))
    uu = float(u[0])
    assert du[0] == pytest.approx(f(Dv[0]) + 3 * delta * uu ** 2 * s, rel=1e-12)   # ∂y/∂u
    assert ddta[0] == pytest.approx(uu ** 3 * s, rel=1e-12)                          # ∂y/∂Δ · ∂Δ/∂dt_active
    assert ddti[0] == pytest.approx(2 * uu ** 3 * s, rel=1e-12)                      # (k-1) = 2
    assert np.allclose(dWB[0], delta * uu ** 3 * f(WC[0])) and np.allclose(dWC[0], delta * uu ** 3 * f(WB[0]))
    assert np.allclose(dA[0], 0.0) and dD[0] == pytest.approx(uu)


# ------------------------------------------- scan with per-event B and C
@pytest.mark.parametrize("with_z", [False, True])
def test_scan_var_reduces_to_depthwise(with_z):
    """B_i = u_i W_B[d], C_i = u_i W_C[d] is the depthwise mode: same out and
    x, and the chain rule through B and C gives the depthwise du, dW_B, dW_C."""
    ch, t, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv, u, dout, z = _bwd_case(2, 4, 70, 5, 0.3, with_z, RNG)
    f8 = lambda v: np.asarray(v, np.float64)
    d = ch % 4
    Bev = f8(u)[:, None] * f8(WB)[d]
    Cev = f8(u)[:, None] * f8(WC)[d]
    ref = orc.scan_fwd(u, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv, z)
    got = orc.scan_var_fwd(u, k, cu, ms, dt_i, dt_a, A, Bev, Cev, Dv, z)
    for a, b in zip(got, ref):
        assert_close(a, b, rtol=1e-12, atol_rel=1e-14, name="fwd")
    out = ref[0]
    rb = orc.scan_bwd(u, k, cu, ms, dt_i, dt_a, A, WB, WC, dout, Dv, z, out if with_z else None)
    du, dA, dBev, dCev, ddti, ddta, dD, dz = orc.scan_var_bwd(u, k, cu, ms, dt_i, dt_a, A, Bev, Cev, dout, Dv, z,
                                                              out if with_z else None)
    du_chain = du + (dBev * f8(WB)[d]).sum(1) + (dCev * f8(WC)[d]).sum(1)
    dWB = np.zeros((4, 5))
    dWC = np.zeros((4, 5))
    np.add.at(dWB, d, dBev * f8(u)[:, None])
    np.add.at(dWC, d, dCev * f8(u)[:, None])
    for name, a, b in [("du", du_chain, rb[0]), ("dA", dA, rb[1]), ("dW_B", dWB, rb[2]), ("dW_C", dWC, rb[3]),
                       ("ddt_idle", ddti, rb[4]), ("ddt_active", ddta, rb[5]), ("dD", dD, rb[6])] + \
            ([("dz", dz, rb[7])] if with_z else []):
        assert_close(a, b, rtol=1e-11, atol_rel=1e-13, name=name)


def test_scan_var_bwd_finite_difference():
    ch, t, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv, u, dout, _ = _bwd_case(1, 2, 40, 3, 0.4, False, RNG)
    E = len(u)
    Bev = RNG.standard_normal((E, 3))
    Cev = RNG.standard_normal((E, 3))
    f8 = lambda v: np.asarray(v, np.float64)
    du, dA, dBev, dCev, ddti, ddta, dD, _ = orc.scan_var_bwd(u, k, cu, ms, dt_i, dt_a, A, Bev, Cev, dout, Dv)

    def loss(uu=f8(u), AA=f8(A), BB=Bev, CC=Cev, ti=f8(dt_i), ta=f8(dt_a)):
        return float(np.dot(orc.scan_var_fwd(uu, k, cu, ms, ti, ta, AA, BB, CC, Dv)[0], f8(dout)))

    eps = 1e-6

    def fd(name, base, idx, grad):
        p_, m_ = base.copy(), base.copy()
        p_[idx] += eps
        m_[idx] -= eps
        num = (loss(**{name: p_}) - loss(**{name: m_})) / (2 * eps)
        assert num == pytest.approx(grad, rel=1e-6, abs=1e-9), (name, idx)

    for i in (0, E // 2, E - 1):
        fd("uu", f8(u), i, du[i])
        fd("BB", Bev, (i, 1), dBev[i, 1])
        fd("CC", Cev, (i, 2), dCev[i, 2])
    fd("AA", f8(A), (1, 2), dA[1, 2])
    fd("ti", f8(dt_i), 1, ddti[1])
    fd("ta", f8(dt_a), 0, ddta[0])


def test_bc_layouts_brute_force_and_adjoint():
    cu = np.array([0, 5, 5, 12, 30], np.int64)
    E, NC, dim, N, T = 30, 4, 2, 3, 4
    legacy = RNG.standard_normal((N, E))
    const = RNG.standard_normal((N, dim))
    n = np.diff(cu)
    tile_off = np.concatenate([[0], np.cumsum((n + T - 1) // T)])[:-1] + 1   # one unused leading tile
    tiled = RNG.standard_normal((int(tile_off[-1] + (n[-1] + T - 1) // T) + 1, N, T))
    for X, kw in [(legacy, {}), (const, {}), (tiled, dict(tile_offsets=tile_off, tile_chunk_size=T))]:
        got = orc.bc_per_event(X, cu, dim, N, **kw)
        want = np.zeros((E, N))
        for c in range(NC):
            for p in range(int(n[c])):
                e = int(cu[c]) + p
                if "tile_offsets" in kw:
                    want[e] = X[tile_off[c] + p // T, :, p % T]
                elif X.shape[1] == E:
                    want[e] = X[:, e]
                else:
                    want[e] = X[:, c % dim]
        assert np.array_equal(got, want)
        G = RNG.standard_normal((E, N))
        back = orc.bc_grad_layout(G, X.shape, cu, dim, **kw)
        assert np.dot(got.ravel(), G.ravel()) == pytest.approx(np.dot(X.ravel(), back.ravel()), rel=1e-12)


def test_pw_grads_finite_difference():
    ch, t, k, cu, ms, dt_i, dt_a, A, WB, WC, Dv, u, dout, _ = _bwd_case(1, 3, 40, 4, 0.4, False, RNG)
    pwB = RNG.standard_normal((3, 3))
    pwC = RNG.standard_normal((3, 3))
    f8 = lambda v: np.asarray(v, np.float64)

    def loss(pB=pwB, pC=pwC, B_=f8(WB), C_=f8(WC)):
        y = orc.scan_fwd(u, k, cu, ms, dt_i, dt_a, A, orc.pw_effective(pB, B_), orc.pw_effective(pC, C_), Dv)[0]
        return float(np.dot(y, f8(dout)))

    r = orc.scan_bwd(u, k, cu, ms, dt_i, dt_a, A, orc.pw_effective(pwB, WB), orc.pw_effective(pwC, WC), dout, Dv)
    dWB, dpwB = orc.pw_grads(pwB, WB, r[2])
    dWC, dpwC = orc.pw_grads(pwC, WC, r[3])
    eps = 1e-6
    for name, base, idx, g in [("pB", pwB, (0, 2), dpwB), ("pC", pwC, (2, 1), dpwC), ("B_", f8(WB), (1, 3), dWB),
                               ("C_", f8(WC), (2, 0), dWC)]:
        p_, m_ = base.copy(), base.copy()
        p_[idx] += eps
        m_[idx] -= eps
        num = (loss(**{name: p_}) - loss(**{name: m_})) / (2 * eps)
        assert num == pytest.approx(g[idx], rel=1e-6, abs=1e-9), name


# --------------------------------------------------- causal conv1d + SiLU
@pytest.mark.parametrize("K,silu,with_bias", [(4, True, True), (4, False, False), (1, True, True), (7, True, False)])
def test_conv1d_matches_torch_conv_and_autograd(K, silu, with_bias):
    B, D, L = 2, 5, 37
    x = RNG.standard_normal((B, D, L))
    w = RNG.standard_normal((D, K))
    bias = RNG.standard_normal(D) if with_bias else None
    dout = RNG.standard_normal((B, D, L))
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    bt = torch.tensor(bias, requires_grad=True) if with_bias else None
    y = torch.nn.functional.conv1d(xt, wt[:, None, :], bt, padding=K - 1, groups=D)[..., :L]
    if silu:
        y = torch.nn.functional.silu(y)
    y.backward(torch.tensor(dout))
    assert_close(orc.conv1d_fwd(x, w, bias, silu), y.detach().numpy(), rtol=1e-12, atol_rel=1e-14, name="out")
    dx, dw, db = orc.conv1d_bwd(x, w, bias, dout, silu)
    assert_close(dx, xt.grad.numpy(), rtol=1e-12, atol_rel=1e-14, name="dx")
    assert_close(dw, wt.grad.numpy(), rtol=1e-12, atol_rel=1e-14, name="dw")
    if with_bias:
        assert_close(db, bt.grad.numpy(), rtol=1e-12, atol_rel=1e-14, name="dbias")


# ---------------------------------------------------------------- restore
def test_restore_fwd_brute_force():
    B, D, L = 2, 3, 45
    mem, ch, t, k, cu, ms = _stream(B, D, L, 0.2, RNG)
    y = RNG.standard_normal(len(ch))
    out = orc.restore_fwd(y, t, cu, D, L)
    for c in range(B * D):
        for s in range(L):
            idx = [e for e in range(cu[c], cu[c + 1]) if t[e] <= s]
            assert out[c // D, s, c % D] == (y[idx[-1]] if idx else 0.0)


def test_restore_bwd_is_adjoint_and_brute_force():
    B, D, L = 2, 4, 70
    mem, ch, t, k, cu, ms = _stream(B, D, L, 0.15, RNG)
    y = RNG.standard_normal(len(ch))
    g = RNG.standard_normal((B, L, D))
    dy = orc.restore_bwd(g, t, cu, D, L)
    assert np.dot(orc.restore_fwd(y, t, cu, D, L).ravel(), g.ravel()) == pytest.approx(np.dot(y, dy), rel=1e-12)
    for e in range(len(ch)):
        c = ch[e]
        nxt = t[e + 1] if e + 1 < cu[c + 1] else L
        assert dy[e] == pytest.approx(g[c // D, t[e]:nxt, c % D].sum(), rel=1e-12)


def test_restore_matches_torch_searchsorted_formulation():
    B, D, L = 2, 3, 64
    mem, ch, t, k, cu, ms = _stream(B, D, L, 0.3, RNG)
    y = RNG.standard_normal(len(ch))
    ref = tp.restore(torch.from_numpy(y), torch.from_numpy(t).long(), torch.from_numpy(ch).long(),
                     torch.from_numpy(cu).long(), D, L)
    assert np.array_equal(orc.restore_fwd(y, t, cu, D, L), ref.numpy())


def test_torch_path_extract_matches_oracle():
    mem = (RNG.random((2, 4, 100)) < 0.2).astype(np.float32)
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem, 0.5)
    tch, tt, tk, tcu, _ = tp.extract(torch.from_numpy(mem), 0.5)
    for a, b in ((ch, tch), (t, tt), (k, tk), (cu, tcu)):
        assert np.array_equal(a, b.numpy())


# ------------------------------------------- conv at the events, spike head
def test_conv_at_events_is_the_dense_conv_read_at_the_events():
    rng = np.random.default_rng(4)
    B, D, L, K = 2, 3, 40, 4
    x = rng.standard_normal((B, D, L))
    w = rng.standard_normal((D, K))
    b = rng.standard_normal(D)
    mask = rng.random((B * D, L)) < 0.3
    ch, t = np.nonzero(mask)
    for silu in (True, False):
        dense = orc.conv1d_fwd(x, w, b, silu).reshape(B * D, L)
        got = orc.conv_at_events(x.reshape(B * D, L), w, b, ch, t, silu)
        assert_close(got, dense[ch, t], rtol=1e-13, atol_rel=1e-14, name="x_events")


def test_conv_bwd_events_matches_autograd_through_the_gather():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    B, D, L, K = 2, 3, 30, 3
    x = rng.standard_normal((B, D, L))
    w = rng.standard_normal((D, K))
    b = rng.standard_normal(D)
    mask = rng.random((B * D, L)) < 0.3
    ch, t = np.nonzero(mask)
    du = rng.standard_normal(len(ch))
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    y = torch.nn.functional.silu(torch.nn.functional.conv1d(xt, wt[:, None, :], bt, padding=K - 1, groups=D)[..., :L])
    y.reshape(B * D, L)[torch.tensor(ch), torch.tensor(t)].mul(torch.tensor(du)).sum().backward()
    dx, dw, db = orc.conv_bwd_events(x, w, b, du, ch, t)
    assert_close(dx, xt.grad.numpy(), rtol=1e-12, atol_rel=1e-13, name="dx")
    assert_close(dw, wt.grad.numpy(), rtol=1e-12, atol_rel=1e-13, name="dw")
    assert_close(db, bt.grad.numpy(), rtol=1e-12, atol_rel=1e-13, name="db")


def test_spike_ste_matches_torch_and_the_dense_extraction():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(6)
    p = rng.random((2, 50, 7)).astype(np.float32)
    s, bits = orc.spike_ste(p, 0.3)
    pt = torch.tensor(p)
    assert np.array_equal(s, ((pt >= 0.3).float() + pt - pt).numpy())
    mem = s.transpose(0, 2, 1).reshape(14, 50)
    assert np.array_equal(bits, mem > 0.5)
