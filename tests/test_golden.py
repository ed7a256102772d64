"""The committed golden fixtures (tests/golden/*.npz) agree with the oracle
and satisfy the path's invariants. Written by tests/golden/make_golden.py;
a change in the oracle that moves any expected value fails here."""
import glob
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, assert_close

GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402

PATH_CASES = [c for c in make_golden.CASES if c != "expand2"]


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_every_case_has_a_fixture():
    have = {os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz"))}
    assert have == set(make_golden.CASES)


@pytest.mark.parametrize("name", list(make_golden.CASES))
def test_fixture_matches_oracle(name):
    want = load(name)
    got = make_golden.CASES[name]()
    assert set(got) == set(want)
    for k, v in want.items():
        g = np.asarray(got[k])
        if v.dtype.kind in "iub":
            assert g.dtype == v.dtype and np.array_equal(g, v), k
        else:
            assert_close(g, v, 1e-6, 1e-7, f"{name}.{k}")


@pytest.mark.parametrize("name", PATH_CASES)
def test_fixture_invariants(name):
    f = load(name)
    B, D, L = f["membrane"].shape
    NC, E = B * D, len(f["t"])
    cu, t, k, ch = f["cu"], f["t"], f["k"], f["ch"]
    assert cu[0] == 0 and cu[-1] == E and np.all(np.diff(cu) >= 0)
    assert np.array_equal(np.diff(cu), f["counts"]) and int(f["max_seqlen"]) == int(f["counts"].max())
    assert np.all(np.diff(ch) >= 0) and np.array_equal(np.repeat(np.arange(NC), f["counts"]), ch)
    for c in range(NC):  # per channel the gaps add up to the time step + 1
        s, e = cu[c], cu[c + 1]
        assert np.array_equal(np.cumsum(k[s:e]), t[s:e] + 1)
    assert f["x"].shape == (NC, max(1, -(-int(f["max_seqlen"]) // 2048)), 2 * f["A"].shape[1])
    # zero-order hold: out is y held from each event to the next, dy sums dout over the same runs
    y = f["y_z"] if "y_z" in f else f["y"]
    assert abs(float((f["out"].astype(np.float64) * f["dout"]).sum()) - float((y.astype(np.float64) * f["dy"]).sum())) \
        <= 1e-4 * float(np.abs(f["out"]).sum() * np.abs(f["dout"]).max() + 1.0)


def test_edges_fixture_covers_the_edge_cases():
    f = load("edges")
    n = f["counts"]
    assert n[0] == 0                    # threshold equality is not an event
    assert n[1] == 1 and f["t"][f["cu"][1]] == 0
    assert n[3] == f["membrane"].shape[2]
    assert f["k"].max() > 64            # a gap longer than one 64-step tile


def test_clamped_fixture_reaches_the_exponent_clamp():
    f = load("clamped")
    d = np.arange(len(f["cu"]) - 1) % f["A"].shape[0]
    kk = f["k"]
    ch = f["ch"]
    delta = f["dt_idle"][d[ch]] * (kk - 1) + f["dt_active"][d[ch]]
    assert (delta[:, None] * f["A"][d[ch]] * 1.4426950408889634).min() < -126


def test_multi_chunk_fixture_has_three_chunks():
    f = load("multi_chunk")
    assert f["x"].shape[1] == 3 and np.abs(f["x"][0, 2]).max() > 0
