"""Writes the golden fixtures of the event path (tests/golden/*.npz).

The reference ships no golden vectors, known-answer tests or fixtures for
this path (its only test is an import smoke test), so the fixtures are
produced by the oracle (oracle/event_path.py), which tests/test_oracle.py
pins against brute force, closed forms, an independent dense formulation and
float64 autograd. Each fixture holds the inputs of one case and the expected
outputs of every stage, forward and backward:

  extract_base_events -> ch, t, k, cu, counts, max_seqlen   (int32, exact)
  gather_fwd          -> u                                   (float32 copy)
  scan_fwd            -> y (or y_z with a z gate), x
  restore_fwd         -> out (B, L, D)
  restore_bwd         -> dy
  scan_bwd            -> du, dA, dW_B, dW_C, ddt_idle, ddt_active, dD (, dz)
  gather_bwd          -> dx (B, D, L)

Expected floats are the float64 oracle results rounded to float32.

Cases (small on purpose, a few hundred KB together):
  cfg0_slice   config 0's generator (membrane N(0,1) > 0.5, ~31% density)
               at B=2, D=8, L=256, N=16
  edges        hand-made channels: none, one event at t=0, one at t=L-1,
               every step, alternating, one long gap (k > 64), 2 events
  multi_chunk  a channel with 4500 events (three 2048-event chunks of the
               saved state x) beside a sparse one, N=8
  clamped      dt large enough that dt*A*log2(e) falls below -126 (the
               reference's exponent clamp), N=4
  z_gate       cfg0-like with the optional z gate, N=16
  expand2      base events of a d_model=4 membrane expanded x2 (indices only)

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import event_path as orc  # noqa: E402

f32 = np.float32


def params(rng, D, N, dt_shift=-2.0, dt_scale=1.0):
    """dt = softplus(N(0,1) - 2), A = -exp(U[ln 1, ln 16]), W = N(0,1)/sqrt(N)."""
    sp = lambda v: np.log1p(np.exp(v))
    return dict(
        dt_idle=(sp(rng.standard_normal(D) + dt_shift) * dt_scale).astype(f32),
        dt_active=(sp(rng.standard_normal(D) + dt_shift) * dt_scale).astype(f32),
        A=(-np.exp(rng.uniform(np.log(1.0), np.log(16.0), (D, N)))).astype(f32),
        W_B=(rng.standard_normal((D, N)) / np.sqrt(N)).astype(f32),
        W_C=(rng.standard_normal((D, N)) / np.sqrt(N)).astype(f32),
        D_skip=np.ones(D, dtype=f32),
    )


def run_path(membrane, x_conv, dout, thr, p, z=None):
    """The full forward and backward of the path through the oracle."""
    B, D, L = membrane.shape
    NC = B * D
    ch, t, k, cu, counts, ms = orc.extract_base_events(membrane, thr)
    u = orc.gather_fwd(x_conv, ch, t).astype(f32)
    args = (p["dt_idle"], p["dt_active"], p["A"], p["W_B"], p["W_C"])
    res = orc.scan_fwd(u, k, cu, ms, *args, D=p["D_skip"], z=z)
    y, x = res[0], res[1]
    y_used = res[2] if z is not None else y
    out = orc.restore_fwd(y_used, t, cu, D, L)
    dy = orc.restore_bwd(dout, t, cu, D, L)
    du, dA, dWB, dWC, ddti, ddta, dD, dz = orc.scan_bwd(u, k, cu, ms, *args, dy, D=p["D_skip"], z=z,
                                                        out=y if z is not None else None)
    dx = orc.gather_bwd(du, ch, t, NC, L).reshape(B, D, L)
    o = dict(membrane=membrane.astype(f32), x_conv=x_conv.astype(f32), dout=dout.astype(f32),
             threshold=np.array(thr, dtype=f32), ch=ch, t=t, k=k, cu=cu, counts=counts,
             max_seqlen=np.array(ms, dtype=np.int32), u=u, y=y.astype(f32), x=x.astype(f32),
             out=out.astype(f32), dy=dy.astype(f32), du=du.astype(f32), dA=dA.astype(f32),
             dW_B=dWB.astype(f32), dW_C=dWC.astype(f32), ddt_idle=ddti.astype(f32),
             ddt_active=ddta.astype(f32), dD=dD.astype(f32), dx=dx.astype(f32))
    o.update({n: v for n, v in p.items()})
    if z is not None:
        o.update(z=z.astype(f32), y_z=res[2].astype(f32), dz=dz.astype(f32))
    return o


def case_cfg0_slice():
    rng = np.random.default_rng(0)
    B, D, L, N = 2, 8, 256, 16
    mem = rng.standard_normal((B, D, L)).astype(f32)
    xc = rng.standard_normal((B, D, L)).astype(f32)
    p = params(rng, D, N)
    dout = rng.standard_normal((B, L, D)).astype(f32)
    return run_path(mem, xc, dout, 0.5, p)


def case_edges():
    rng = np.random.default_rng(1)
    B, D, L, N = 1, 8, 130, 4
    mem = np.zeros((B, D, L), dtype=f32)
    mem[0, 1, 0] = 1.0                 # one event at t = 0
    mem[0, 2, L - 1] = 1.0             # one event at the last step
    mem[0, 3, :] = 1.0                 # every step (k = 1 throughout)
    mem[0, 4, ::2] = 1.0               # alternating (k = 2)
    mem[0, 5, [3, 100]] = 1.0          # a gap of 97 steps (past a 64-step tile)
    mem[0, 6, [63, 64]] = 1.0          # events on both sides of a tile edge
    mem[0, 7, [0, 65, 129]] = 1.0      # tile-crossing runs
    mem[0, 0, :] = 0.5                 # equal to the threshold: no event (strict >)
    xc = rng.standard_normal((B, D, L)).astype(f32)
    p = params(rng, D, N)
    dout = rng.standard_normal((B, L, D)).astype(f32)
    return run_path(mem, xc, dout, 0.5, p)


def case_multi_chunk():
    rng = np.random.default_rng(2)
    B, D, L, N = 1, 2, 4500, 8
    mem = np.zeros((B, D, L), dtype=f32)
    mem[0, 0, :] = 1.0
    mem[0, 1, :] = (rng.random(L) < 0.05).astype(f32)
    xc = rng.standard_normal((B, D, L)).astype(f32)
    p = params(rng, D, N, dt_shift=-5.0)   # slow decay: state carries across chunks
    dout = rng.standard_normal((B, L, D)).astype(f32)
    return run_path(mem, xc, dout, 0.5, p)


def case_clamped():
    rng = np.random.default_rng(3)
    B, D, L, N = 2, 2, 300, 4
    mem = (rng.random((B, D, L)) < 0.1).astype(f32)
    xc = rng.standard_normal((B, D, L)).astype(f32)
    p = params(rng, D, N, dt_shift=2.0, dt_scale=3.0)  # Δ·A·log2e well below -126 for long gaps
    dout = rng.standard_normal((B, L, D)).astype(f32)
    return run_path(mem, xc, dout, 0.5, p)


def case_z_gate():
    rng = np.random.default_rng(4)
    B, D, L, N = 2, 4, 128, 16
    mem = rng.standard_normal((B, D, L)).astype(f32)
    xc = rng.standard_normal((B, D, L)).astype(f32)
    p = params(rng, D, N)
    dout = rng.standard_normal((B, L, D)).astype(f32)
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem, 0.5)
    z = rng.standard_normal(len(t)).astype(f32)
    return run_path(mem, xc, dout, 0.5, p, z=z)


def case_expand2():
    rng = np.random.default_rng(5)
    B, Dm, L, expand = 2, 4, 96, 2
    mem = (rng.random((B, Dm, L)) < 0.2).astype(f32)
    ch, t, k, cu, counts, ms = orc.extract_base_events(mem, 0.5)
    ech, et, ek, ecu, ems = orc.expand_base_events(ch, t, k, cu, B, Dm, expand)
    return dict(membrane=mem, threshold=np.array(0.5, dtype=f32), expand=np.array(expand, dtype=np.int32),
                ch=ch, t=t, k=k, cu=cu, e_ch=ech, e_t=et, e_k=ek, e_cu=ecu,
                e_max_seqlen=np.array(ems, dtype=np.int32))


CASES = {
    "cfg0_slice": case_cfg0_slice,
    "edges": case_edges,
    "multi_chunk": case_multi_chunk,
    "clamped": case_clamped,
    "z_gate": case_z_gate,
    "expand2": case_expand2,
}


def main():
    for name, fn in CASES.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
