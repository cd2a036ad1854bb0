"""MI355X-native selective scan -- drop-in for zouyuanqing/mamba-windows-cuda.

Exports the reference's package surface (mamba_windows_cuda/__init__.py:1-4)
plus the checkpoint-level module of selective_scan_cuda_ext.py.
"""
from .mamba_cuda import SelectiveScanCuda, selective_scan_ref
from .pscan import parallel_scan_fn, parallel_scan_ref
from .selective_scan_cuda_ext import FusedSelectiveScan

__all__ = ["SelectiveScanCuda", "parallel_scan_fn", "parallel_scan_ref", "FusedSelectiveScan",
           "selective_scan_ref"]
__version__ = "0.5.0+mi355x"
