"""Build libbcm_event_scan.so (HIP, gfx950) in-tree with hipcc.

Usage: python -m bc_mamba_amd.build  (or bc_mamba_amd.build.build())

The library is a plain C-ABI shared object: no torch headers, no pybind11.
It links against the HIP runtime by SONAME (libamdhip64.so.7); inside a
process that imported torch first, the loader binds it to the HIP runtime
torch already loaded, so streams and device pointers are shared.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIBDIR = os.path.join(HERE, "lib")
BUILDDIR = os.path.join(HERE, "lib", "_obj")
LIBNAME = "libbcm_event_scan.so"
ARCH = os.environ.get("BCM_OFFLOAD_ARCH", "gfx950")

SOURCES = ["abi.hip", "extract.hip", "scan.hip", "scan_sl.hip", "scan_var.hip", "restore.hip", "restore_proj.hip", "conv.hip"]

# Packed FP32 (v_pk_*_f32) generation is switched off for all device code.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-unused-command-line-argument",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build bc_mamba_amd)")


def _compile(src):
    obj = os.path.join(BUILDDIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj, r.stderr


def build(verbose=False):
    """Compile every HIP source and link lib/libbcm_event_scan.so. Returns its path."""
    os.makedirs(BUILDDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        results = list(ex.map(_compile, SOURCES))
    objs = [o for o, _ in results]
    if verbose:
        for _, err in results:
            if err.strip():
                print(err, file=sys.stderr)
    out = os.path.join(LIBDIR, LIBNAME)
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
