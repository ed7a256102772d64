"""Stage markers of the event path (the reference's no-op `cuda_stage`,
spike_mamba/runtime_breakdown.py:13-15). Here each stage is a
torch.profiler.record_function range, which rocprofv3 / torch.profiler show
next to the HIP kernels it launches."""
from contextlib import contextmanager

import torch

__all__ = ["cuda_stage"]


@contextmanager
def cuda_stage(name):
    with torch.profiler.record_function(name):
        yield
