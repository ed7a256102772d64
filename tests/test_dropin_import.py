"""The drop-in modules import under the reference's bare module names, as the
reference's own import check does (reference tests/test_import.py:10-22):
with bc_mamba_amd/ on sys.path, `import selective_scan_cuda` and friends
resolve to this package's modules. Runs in a subprocess so the bare-name
modules do not mix with the package imports of the other tests."""
import os
import subprocess
import sys

from conftest import ROOT

SCRIPT = r"""
import sys
from pathlib import Path
pkg = Path(sys.argv[1])
sys.path.insert(0, str(pkg))
import e_model, selective_scan_interface, selective_scan_cuda, extract_events_cuda, restore_dense_cuda_nodecay
assert e_model.Mamba.__name__ == "Mamba"
assert hasattr(selective_scan_interface, "selective_scan_flat_ch_fn")
assert hasattr(selective_scan_interface, "SelectiveScanFlatChFn")
assert hasattr(restore_dense_cuda_nodecay, "restore_dense_fwd") and hasattr(restore_dense_cuda_nodecay, "restore_dense_bwd")
for name in ("extract_base_events", "expand_base_events", "gather_events_fwd", "gather_events_bwd", "extract_events"):
    assert hasattr(extract_events_cuda, name), name
for name in ("fwd_flat_ch", "bwd_flat_ch"):
    assert hasattr(selective_scan_cuda, name), name
for ext in (selective_scan_cuda, extract_events_cuda, restore_dense_cuda_nodecay):
    assert Path(ext.__file__).resolve().parent == pkg.resolve(), ext.__file__
print("drop-in import OK")
"""


def test_reference_module_names_resolve_to_this_package():
    r = subprocess.run([sys.executable, "-c", SCRIPT, os.path.join(ROOT, "bc_mamba_amd")],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=300)
    assert r.returncode == 0 and b"drop-in import OK" in r.stdout, r.stdout.decode()[-2000:]
