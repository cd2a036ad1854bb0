"""First-order linear recurrence H_t = A_t*H_{t-1} + X_t -- the drop-in for
``mamba_windows_cuda.pscan`` (zouyuanqing/mamba-windows-cuda, pscan.py:1-171).

``parallel_scan_fn(A, X)`` runs the single-pass decoupled look-back scan of
libmwc_ssm.so on the GPU with the semantics of ``parallel_scan_ref``
(H_0 = X_0, A_0 unused) for any L -- the reference's ``PScan`` needs a power
of two and its up/down sweeps are wrong for L >= 4 (pscan.py:46-71). Inputs
are (B, D, L, N) with the scan over dim 2, or (B, L, C) with the scan over
dim 1; fp32 or fp16 storage, fp32 accumulation. The backward is the exact
adjoint (pscan.py:97-136 raises a shape error whenever D != L).
"""
from __future__ import annotations

import torch

from . import ops


class PScan(torch.autograd.Function):
    """Autograd function behind ``parallel_scan_fn`` (pscan.py:16-136)."""

    @staticmethod
    def forward(ctx, A_in, X_in):
        H = ops.pscan_forward(A_in, X_in)
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
            ctx.save_for_backward(A_in, H)
        return H

    @staticmethod
    def backward(ctx, grad_output):
        A_in, H = ctx.saved_tensors
        dA, dX = ops.pscan_backward(A_in, H, grad_output)
        return dA, dX


def parallel_scan_fn(A, X):
    """H with H_0 = X_0 and H_t = A_t*H_{t-1} + X_t along the sequence axis (pscan.py:139-150)."""
    return PScan.apply(A, X)


def pscan_check():
    """Wait for the scans enqueued so far and raise RuntimeError if a bounded look-back wait in one of
    them gave up (its outputs are then NaN). Not in the reference, whose PScan has no waits: scan
    calls report such a failure without waiting, at the first call after it finished."""
    ops.pscan_check()


def parallel_scan_ref(A, X):
    """Sequential reference scan (pscan.py:153-171): plain PyTorch, any device,
    accumulating in the input dtype. Accepts (B, D, L, N) or (B, L, C)."""
    H = torch.zeros_like(X)
    H[..., 0, :] = X[..., 0, :]
    for t in range(1, X.shape[-2]):
        H[..., t, :] = A[..., t, :] * H[..., t - 1, :] + X[..., t, :]
    return H
