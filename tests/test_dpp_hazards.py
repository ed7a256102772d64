"""DPP read-after-VALU-write hazards in this build's own gfx950 assembly.

A DPP instruction reads its first source through the DPP crossbar, which on
gfx9-family parts needs two wait states after a VALU instruction wrote that
register (`s_nop 1`, or two independent instructions in between). The
compiler inserts them for the DPP instructions it emits itself, but not for
the inline-asm ones of the state-lane scans (`fmac_bcast`, `tab16` in
csrc/scan_sl.hip), which rely on their sources having been written well
before. A register copy placed right before one of them by the register
allocator would read a stale value without any error, so this test compiles
scan_sl.hip to assembly and checks every DPP instruction in it.

The walk back from a DPP instruction goes through labels as if the block
above fell through (the paths that enter by a branch are not followed)."""
import os
import re
import shutil
import subprocess

import pytest

from conftest import ROOT

CSRC = os.path.join(ROOT, "bc_mamba_amd", "csrc")


def _regs(op):
    """VGPR numbers of an operand: v12 -> {12}, v[4:7] -> {4, 5, 6, 7}."""
    m = re.fullmatch(r"v(\d+)", op)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def _parse(line):
    """(mnemonic, [operands]) of an instruction line, or None."""
    s = line.split(";", 1)[0].strip()
    if not s or s.startswith(".") or s.endswith(":"):
        return None
    parts = s.split(None, 1)
    ops = [o.strip().split()[0] for o in parts[1].split(",")] if len(parts) > 1 else []
    return parts[0], ops


def dpp_hazards(asm):
    """[(function, line number, text)] of DPP instructions whose first source
    was written by a VALU instruction fewer than two wait states before."""
    found, hist, fn = [], [], "?"
    for no, line in enumerate(asm.splitlines(), 1):
        m = re.match(r"^(_Z\w+):", line)
        if m:
            fn, hist = m.group(1), []
            continue
        p = _parse(line)
        if p is None:
            continue
        mn, ops = p
        if mn.endswith("_dpp") and len(ops) >= 2:
            src = _regs(ops[1])
            ws = 0
            for pm, pops in reversed(hist):
                if ws >= 2:
                    break
                if pm == "s_nop":
                    ws += int(pops[0], 0) + 1
                    continue
                if pm.startswith("v_") and pops and _regs(pops[0]) & src:
                    found.append((fn, no, line.strip()))
                    break
                ws += 1
        hist = (hist + [(mn, ops)])[-4:]
    return found


def test_checker_finds_a_planted_hazard():
    bad = "_Zk:\n\tv_mov_b32_e32 v5, v6\n\tv_fmac_f32_dpp v1, v5, v2 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
    assert len(dpp_hazards(bad)) == 1
    near = "_Zk:\n\tv_mov_b32_e32 v5, v6\n\ts_mov_b32 s0, 0\n\tv_add_u32_dpp v1, v5, v2 row_newbcast:1\n"
    assert len(dpp_hazards(near)) == 1  # one wait state is not enough
    ok = "_Zk:\n\tv_mov_b32_e32 v5, v6\n\ts_nop 1\n\tv_fmac_f32_dpp v1, v5, v2 row_newbcast:3\n"
    assert dpp_hazards(ok) == []
    ok2 = "_Zk:\n\tv_mov_b32_e32 v[4:5], v[6:7]\n\tv_add_f32_e32 v9, v9, v9\n\tv_mul_f32_e32 v8, v8, v8\n" \
          "\tv_mov_b32_dpp v1, v5 row_newbcast:2\n"
    assert dpp_hazards(ok2) == []
    wide = "_Zk:\n\tv_lshl_add_u64 v[4:5], v[6:7], 0, v[2:3]\n\tv_mov_b32_dpp v1, v5 row_newbcast:2\n"
    assert len(dpp_hazards(wide)) == 1


def test_state_lane_scans_have_no_dpp_hazard(tmp_path):
    hipcc = next((c for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc"))
                  if c and os.path.exists(c)), None)
    if hipcc is None:
        pytest.skip("hipcc not found")
    from bc_mamba_amd.build import HIPCC_FLAGS, INCLUDE
    out = tmp_path / "scan_sl.s"
    cmd = [hipcc, *HIPCC_FLAGS, "-I", INCLUDE, "-I", CSRC, "--cuda-device-only", "-S",
           os.path.join(CSRC, "scan_sl.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    assert asm.count("v_fmac_f32_dpp") > 100  # the inline-asm broadcasts are there to be checked
    hz = dpp_hazards(asm)
    assert not hz, "\n".join(f"{f}:{n}: {t}" for f, n, t in hz[:20])
