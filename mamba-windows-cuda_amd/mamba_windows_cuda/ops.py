"""Host wrappers (one call = one enqueue on the current HIP stream). Tensors are borrowed; outputs
and scratch come from the torch caching allocator.

The selective-scan wrappers (checks, forward, backward, decode step) call the raw PyTorch operators
of libmwc_torch.so (csrc/torch_ops.cpp): the reference host wrapper's contract and messages
(``selective_scan_cuda_forward_with_state``, mamba_windows_cuda/mamba_cuda.py:281-326; device,
dtype, last-dim contiguity, N == 16 widened to N in {8, 16, 32, 64}, ranks and shapes, then the
optional h_prev) are checked in C++, and violations raise RuntimeError before any device work is
queued. The parallel-scan wrappers call the C ABI through ctypes and keep the status words of recent
scans.
"""
from __future__ import annotations

import collections
import threading

import torch

from . import _lib

NSTATE = 16
# state counts the kernels are built for (the reference builds N=16 only)
NSTATES = (8, 16, 32, 64)


STORAGE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _dtype_code(t: torch.Tensor) -> int:
    return {torch.float16: _lib.MWC_DTYPE_F16, torch.bfloat16: _lib.MWC_DTYPE_BF16}.get(t.dtype, _lib.MWC_DTYPE_F32)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device):
    """The current HIP stream of `dev` (a raw hipStream_t as an int)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


class _on_device:
    """Makes `dev` the current HIP device for a launch; costs nothing when it already is (the usual
    case), unlike ``torch.cuda.device``, which switches and restores every time."""

    __slots__ = ("idx", "prev")

    def __init__(self, dev: torch.device):
        self.idx = dev.index

    def __enter__(self):
        self.prev = torch.cuda.current_device()
        if self.prev != self.idx:
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev != self.idx:
            torch.cuda.set_device(self.prev)
        return False


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def check_ssm_inputs(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, *, require_device=True):
    """Raise RuntimeError unless the inputs satisfy the reference's contract (the checks of
    torch.ops.mwc.ssm_scan, which every scan call runs; require_device=False skips the device-type
    checks)."""
    _lib.torch_ops().check_ssm_inputs(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, require_device)


def check_transforms(u, delta_bias=None, z=None):
    """The optional elementwise transforms around the scan: delta_bias (D,), z (B, L, D)."""
    _lib.torch_ops().check_transforms(u, delta_bias, z)


def ssm_forward_xf(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, *, delta_bias=None, delta_softplus=False,
                   z=None, want_out=True, want_ungated=False, want_h_last=True, want_ckpt=False):
    """Fused forward with the optional transforms (delta' = softplus(delta + delta_bias),
    out_z = out * silu(z)). Returns (out_z or out, ungated out or None, h_last or None, ckpt or None).

    ckpt is fp32 (B, ceil(L/16), D, N): the state before every 16th step,
    which the backward restarts from. Checks, allocation and launch are torch.ops.mwc.ssm_fwd's."""
    return tuple(_lib.torch_ops().ssm_fwd(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, delta_bias, bool(delta_softplus),
                                          z, want_out, want_ungated, want_h_last, want_ckpt))


def ssm_forward(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, *, want_out=True, want_h_last=True,
                want_ckpt=False):
    """Fused forward. Returns (out or None, h_last or None, ckpt or None)."""
    out, _, h_last, ckpt = ssm_forward_xf(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, want_out=want_out,
                                          want_h_last=want_h_last, want_ckpt=want_ckpt)
    return out, h_last, ckpt


def ssm_backward_xf(u, delta, A, B_ssm, C_ssm, D_ssm, dout, ckpt, dh_last=None, want_dh_prev=False, *,
                    delta_bias=None, delta_softplus=False, z=None, out_ungated=None):
    """Fused backward with the optional transforms. With z, dout is the gradient of the gated
    output and out_ungated the forward's ungated output. Returns
    (du, ddelta, dA, dB, dC, dD, dh_prev or None, ddelta_bias or None, dz or None), in u's dtype.
    Checks, allocation and launch are torch.ops.mwc.ssm_bwd's."""
    return tuple(_lib.torch_ops().ssm_bwd(u, delta, A, B_ssm, C_ssm, D_ssm, dout, ckpt, dh_last, bool(want_dh_prev),
                                          delta_bias, bool(delta_softplus), z, out_ungated))


def ssm_backward(u, delta, A, B_ssm, C_ssm, D_ssm, dout, ckpt, dh_last=None, want_dh_prev=False):
    """Fused backward. Returns (du, ddelta, dA, dB, dC, dD, dh_prev or None), in u's dtype."""
    return ssm_backward_xf(u, delta, A, B_ssm, C_ssm, D_ssm, dout, ckpt, dh_last, want_dh_prev)[:7]


def ssm_step(u, delta, A, B_ssm, C_ssm, D_ssm, h, *, delta_bias=None, delta_softplus=False, z=None,
             out_state=None):
    """One decode step: u, delta, z (B, D); A (D, N); B_ssm, C_ssm (B, N); D_ssm (D,); h (B, D, N).
    Returns (out (B, D) -- gated by silu(z) when z is given --, h_new (B, D, N)). out_state, when
    given, receives h_new and may be h itself (in-place update). torch.ops.mwc.ssm_step."""
    return tuple(_lib.torch_ops().ssm_step(u, delta, A, B_ssm, C_ssm, D_ssm, h, z, delta_bias, bool(delta_softplus),
                                           out_state))


def _scan_view(x: torch.Tensor):
    """(B, D, L, N) -> (B*D, L, N) and (B, L, C) -> itself; the scan runs over dim -2."""
    if x.dim() == 4:
        b, d, l, n = x.shape
        return x.reshape(b * d, l, n)
    if x.dim() == 3:
        return x
    raise RuntimeError("parallel scan inputs must be 4D (B, D, L, N) or 3D (B, L, C)")


def _check_scan(*ts):
    for t in ts:
        _require(t.is_cuda, "parallel_scan_fn inputs must be CUDA tensors")
        _require(t.dtype in STORAGE_DTYPES, "parallel_scan_fn supports float32/float16 (or bfloat16)")
        _require(t.dtype == ts[0].dtype and tuple(t.shape) == tuple(ts[0].shape),
                 "parallel_scan_fn inputs must share dtype and shape")
        _require(t.device == ts[0].device, "parallel_scan_fn inputs must share a device")


# Status words of recent scans, read without waiting for the GPU: each call enqueues a copy of its
# scan's status word into pinned host memory plus an event, and every later call (or pscan_check())
# looks at the words whose events have completed. A bounded look-back wait that gave up (its tiles'
# outputs are NaN) is so reported by the first scan call, or pscan_check(), after it finished.
_pending_status = collections.deque()  # (event, pinned int32 word, what)
_pending_lock = threading.Lock()
_MAX_PENDING = 256


def _pscan_status(L_, ws, nbytes, nseq, L, nc, dev, what):
    """Enqueue the read of the status word of the scan just enqueued (skipped while a graph is being
    captured: the word is then never read)."""
    if torch.cuda.is_current_stream_capturing():
        return
    word = torch.empty(1, dtype=torch.int32, pin_memory=True)
    with _on_device(dev):
        st = L_.mwc_pscan_status_async(ws.data_ptr(), nbytes, nseq, L, nc, word.data_ptr(), _stream(dev))
        _lib.check(st, what)
        ev = torch.cuda.Event()
        ev.record()
    with _pending_lock:
        _pending_status.append((ev, word, what))
        full = len(_pending_status) > _MAX_PENDING
    if full:
        _drain_status(wait_oldest=True)


def _drain_status(wait_all=False, wait_oldest=False):
    """Retire the status words whose scans have finished (all of them, waiting, with wait_all) and
    raise RuntimeError if one of them reports a wait that gave up. Nothing is queried while a graph
    is being captured (event queries are not allowed then)."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        return
    failed = None
    first = True
    with _pending_lock:
        while _pending_status:
            ev, word, what = _pending_status[0]
            if wait_all or (wait_oldest and first):
                ev.synchronize()
            elif not ev.query():
                break
            first = False
            _pending_status.popleft()
            if int(word[0]) != 0 and failed is None:
                failed = what
    if failed is not None:
        raise RuntimeError(f"{failed} failed: MWC_ERR_INCOMPLETE: a look-back wait of an earlier parallel scan "
                           "ran out of spins, so the affected tiles' outputs are NaN")


def pscan_check():
    """Wait for every scan enqueued so far and raise RuntimeError (MWC_ERR_INCOMPLETE) if one of them
    gave up a look-back wait. Scan calls already report such a failure once it has finished, at the
    next call; this makes the report immediate."""
    _drain_status(wait_all=True)


def pscan_forward(A, X):
    _check_scan(A, X)
    _drain_status()
    A, X = A.contiguous(), X.contiguous()
    a3, x3 = _scan_view(A), _scan_view(X)
    H = torch.empty_like(X)
    h3 = _scan_view(H)
    nseq, L, nc = x3.shape
    L_ = _lib.lib()
    nbytes = L_.mwc_pscan_workspace_size(nseq, L, nc)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=X.device)
    with _on_device(X.device):
        st = L_.mwc_pscan_fwd(_dtype_code(X), a3.data_ptr(), x3.data_ptr(), h3.data_ptr(), nseq, L, nc,
                              ws.data_ptr(), nbytes, _stream(X.device))
    _lib.check(st, "mwc_pscan_fwd")
    _pscan_status(L_, ws, nbytes, nseq, L, nc, X.device, "mwc_pscan_fwd")
    return H


def pscan_backward(A, H, dH):
    _check_scan(A, H, dH)
    _drain_status()
    A, H, dH = A.contiguous(), H.contiguous(), dH.contiguous()
    dA = torch.empty_like(A)
    dX = torch.empty_like(A)
    a3, h3, g3, da3, dx3 = (_scan_view(t) for t in (A, H, dH, dA, dX))
    nseq, L, nc = h3.shape
    L_ = _lib.lib()
    nbytes = L_.mwc_pscan_workspace_size(nseq, L, nc)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=H.device)
    with _on_device(H.device):
        st = L_.mwc_pscan_bwd(_dtype_code(H), a3.data_ptr(), h3.data_ptr(), g3.data_ptr(), da3.data_ptr(),
                              dx3.data_ptr(), nseq, L, nc, ws.data_ptr(), nbytes, _stream(H.device))
    _lib.check(st, "mwc_pscan_bwd")
    _pscan_status(L_, ws, nbytes, nseq, L, nc, H.device, "mwc_pscan_bwd")
    return dA, dX
