"""TEST INFRASTRUCTURE ONLY: plain-torch restatements of the reference's
sequential CPU path, used (a) to pin the C oracle through torch autograd and
(b) as bench.py's ``cpu_baseline`` ("port" of the reference's PyTorch path).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module. Nothing here is reference source: each function is
written from the semantics of the cited reference function.

* ``selective_scan_seq``   -- semantics of ``selective_scan_ref``
  (mamba_windows_cuda/mamba_cuda.py:875-946): per-step loop over L of
  h = exp(delta*A)*h + delta*u*B, then y = sum_n C*h + D*u.
* ``selective_scan_closed`` -- the cumsum closed form used by the reference's
  own tests (mamba_windows_cuda/tests/test_selective_scan.py:8-36):
  h_t = e^{A S_t} (h_prev + sum_{s<=t} e^{-A S_s} delta_s u_s B_s), S = cumsum(delta).
* ``pscan_seq``            -- semantics of ``parallel_scan_ref``
  (mamba_windows_cuda/pscan.py:153-171).
"""
from __future__ import annotations

import torch


def selective_scan_seq(u, delta, A, B, C, D, h_prev=None):
    """Sequential scan with autograd support. Shapes: u, delta (B,L,D); A (D,N);
    B, C (B,L,N); D (D,); h_prev (B,D,N). Returns (out (B,L,D), h_last (B,D,N))."""
    bsz, L, dm = u.shape
    n = A.shape[1]
    h = torch.zeros(bsz, dm, n, dtype=u.dtype, device=u.device) if h_prev is None else h_prev
    ys = []
    for t in range(L):
        dt = delta[:, t, :].unsqueeze(-1)                    # (B,D,1)
        dA = torch.exp(dt * A.unsqueeze(0))                  # (B,D,N)
        dBu = dt * u[:, t, :].unsqueeze(-1) * B[:, t, :].unsqueeze(1)
        h = dA * h + dBu
        ys.append((h * C[:, t, :].unsqueeze(1)).sum(-1) + D * u[:, t, :])
    return torch.stack(ys, dim=1), h


def selective_scan_vectorized(u, delta, A, B, C, D, h_prev=None):
    """The same recurrence arranged like the reference's ``selective_scan_ref``:
    dA and dBu materialised over (B,D,N,L) with einsum/broadcast, then the
    per-step loop (mamba_cuda.py:910-929). Used as the timed CPU baseline."""
    bsz, L, dm = u.shape
    n = A.shape[1]
    u_t, d_t = u.transpose(1, 2), delta.transpose(1, 2)      # (B,D,L)
    B_t, C_t = B.transpose(1, 2), C.transpose(1, 2)          # (B,N,L)
    h = torch.zeros(bsz, dm, n, dtype=u.dtype, device=u.device) if h_prev is None else h_prev
    dA = torch.exp(d_t.unsqueeze(2) * A.view(1, dm, n, 1))   # (B,D,N,L)
    dBu = (d_t * u_t).unsqueeze(2) * B_t.unsqueeze(1)        # (B,D,N,L)
    hs = []
    h = h.unsqueeze(-1)
    for t in range(L):
        h = dA[..., t:t + 1] * h + dBu[..., t:t + 1]
        hs.append(h)
    hs = torch.cat(hs, dim=-1)                               # (B,D,N,L)
    y = (C_t.unsqueeze(1) * hs).sum(2) + u_t * D.view(1, -1, 1)
    return y.transpose(1, 2), h.squeeze(-1)


def selective_scan_closed(u, delta, A, B, C, D, h_prev=None):
    """Closed form via cumulative sums (stable only while |A*cumsum(delta)| is small)."""
    bsz, L, dm = u.shape
    n = A.shape[1]
    if h_prev is None:
        h_prev = torch.zeros(bsz, dm, n, dtype=u.dtype)
    S = torch.cumsum(delta.transpose(1, 2), dim=2)           # (B,D,L)
    E = S.unsqueeze(2) * A.view(1, dm, n, 1)                 # (B,D,N,L)
    dBu = (delta * u).transpose(1, 2).unsqueeze(2) * B.transpose(1, 2).unsqueeze(1)
    h = torch.exp(E) * (h_prev.unsqueeze(-1) + torch.cumsum(torch.exp(-E) * dBu, dim=3))
    y = (C.transpose(1, 2).unsqueeze(1) * h).sum(2) + u.transpose(1, 2) * D.view(1, -1, 1)
    return y.transpose(1, 2), h[..., -1]


def pscan_seq(A, X):
    """H_0 = X_0; H_t = A_t*H_{t-1} + X_t along dim -2 (autograd-capable)."""
    hs = [X[..., 0, :]]
    for t in range(1, X.shape[-2]):
        hs.append(A[..., t, :] * hs[-1] + X[..., t, :])
    return torch.stack(hs, dim=-2)
