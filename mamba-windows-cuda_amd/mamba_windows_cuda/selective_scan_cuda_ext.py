"""``FusedSelectiveScan(checkpoint_lvl)`` -- the drop-in for
``mamba_windows_cuda.selective_scan_cuda_ext`` (zouyuanqing/mamba-windows-cuda,
selective_scan_cuda_ext.py:562-677), whose own CUDA source does not compile.
The API and the meaning of the knob are kept; the work is the same fused
gfx950 forward/backward as ``SelectiveScanCuda``:

* ``checkpoint_lvl=0`` -- save: the forward stores fp32 state checkpoints
  (every 16 steps) for the backward;
* ``checkpoint_lvl=1`` -- recompute: only the inputs are kept; the backward
  rebuilds the checkpoints with a state-only forward pass first.
"""
from __future__ import annotations

import torch

from .mamba_cuda import _backward_impl, _forward_impl, _ssm_scan


class FusedSelectiveScanFunction(torch.autograd.Function):
    """(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, checkpoint_lvl=0) -> (out, h_last), on the
    Python host path; FusedSelectiveScan calls the C++ operator torch.ops.mwc.ssm_scan instead."""

    @staticmethod
    def forward(ctx, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, checkpoint_lvl=0):
        return _forward_impl(ctx, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, checkpoint_lvl)

    @staticmethod
    def backward(ctx, dout, dh_last):
        return (*_backward_impl(ctx, dout, dh_last)[:7], None)


class FusedSelectiveScan(torch.nn.Module):
    """Fused selective scan with a checkpoint level (0 = save, 1 = recompute)."""

    def __init__(self, checkpoint_lvl: int = 0):
        super().__init__()
        if checkpoint_lvl not in (0, 1):
            raise ValueError(f"checkpoint_lvl must be 0 or 1 (got {checkpoint_lvl})")
        self.checkpoint_lvl = checkpoint_lvl

    def forward(self, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None):
        return _ssm_scan(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, self.checkpoint_lvl, None, None, False)[0]

    def forward_with_state(self, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None):
        return _ssm_scan(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, self.checkpoint_lvl, None, None, False)
