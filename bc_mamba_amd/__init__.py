"""bc_mamba_amd - MI355X-native (gfx950 HIP) event-sparse selective-scan path
of BC_mamba: event extraction, flat per-channel selective scan and
zero-order-hold restore, forward and backward.

Drop-in modules (same names as the reference's extension modules and
Python files; put this directory on sys.path to import them by those names):
  selective_scan_cuda         fwd_flat_ch / bwd_flat_ch
  extract_events_cuda         extract_base_events / expand_base_events /
                              gather_events_fwd / gather_events_bwd / extract_events
  restore_dense_cuda_nodecay  restore_dense_fwd / restore_dense_bwd
  selective_scan_interface    SelectiveScanFlatChFn / selective_scan_flat_ch_fn
  e_model                     RestoreDenseFn / GatherEventsFn / TwoLevelDelta / Mamba

All compute runs in libbcm_event_scan.so (C ABI: include/bcm_event_scan.h).
"""
import os

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))

__all__ = ["PACKAGE_DIR"]
