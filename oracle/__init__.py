"""Test infrastructure: CPU oracles of the BC_mamba event path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker or the timed CPU baseline; the product
package bc_mamba_amd never does.
"""
