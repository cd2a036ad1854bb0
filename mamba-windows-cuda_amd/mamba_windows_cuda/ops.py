"""Validated host wrappers over the C ABI (one call = one enqueue on the
current HIP stream). Tensors are borrowed; outputs and scratch come from the
torch caching allocator.

The validation restates the reference host wrapper's contract and messages
(``selective_scan_cuda_forward_with_state``, mamba_windows_cuda/mamba_cuda.py:
281-326): device, dtype (fp32/fp16, all equal), last-dim contiguity, N == 16
(widened here to N in {8, 16, 32, 64}), ranks and shapes, then the optional h_prev. Violations raise RuntimeError
before any device work is queued.
"""
from __future__ import annotations

import collections
import functools
import os
import threading

import torch

from . import _lib

NSTATE = 16
# state counts the kernels are built for (the reference builds N=16 only)
NSTATES = (8, 16, 32, 64)


STORAGE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _dtype_code(t: torch.Tensor) -> int:
    return {torch.float16: _lib.MWC_DTYPE_F16, torch.bfloat16: _lib.MWC_DTYPE_BF16}.get(t.dtype, _lib.MWC_DTYPE_F32)


def _ptr(t):
    return None if t is None else t.data_ptr()


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
    """Raise RuntimeError unless the inputs satisfy the reference's contract."""
    # (messages are formatted only on failure: these checks run on every call)
    named = (("u", u), ("delta", delta), ("A", A), ("B_ssm", B_ssm), ("C_ssm", C_ssm), ("D_ssm", D_ssm))
    if require_device:
        for name, t in named:
            if not t.is_cuda:
                raise RuntimeError(f"{name} must be a CUDA tensor")
    # bfloat16 is accepted in addition to the reference's float32/float16 (storage only, fp32 math)
    _require(u.dtype in STORAGE_DTYPES, "u must be float32/float16 (or bfloat16)")
    for name, t in named[1:]:
        if t.dtype != u.dtype:
            raise RuntimeError(f"{name} dtype must match u dtype")
    for name, t in named:
        if not (t.dim() == 0 or t.stride(-1) == 1 or t.size(-1) == 1):
            raise RuntimeError(f"{name} must be contiguous in the last dimension")
    _require(A.dim() == 2, "A must be 2D (dim, state)")
    _require(A.size(1) in NSTATES, "Only N=16 (or 8, 32, 64) is supported")
    n = A.size(1)
    _require(u.dim() == 3, "u must be 3D (batch, seqlen, dim)")
    _require(delta.dim() == 3, "delta must be 3D (batch, seqlen, dim)")
    _require(B_ssm.dim() == 3, "B_ssm must be 3D (batch, seqlen, state)")
    _require(C_ssm.dim() == 3, "C_ssm must be 3D (batch, seqlen, state)")
    _require(D_ssm.dim() == 1, "D_ssm must be 1D (dim)")
    bsz, L, dm = u.shape
    _require(tuple(delta.shape) == (bsz, L, dm), "delta shape mismatch")
    _require(tuple(A.shape) == (dm, n), "A shape mismatch")
    _require(tuple(B_ssm.shape) == (bsz, L, n), "B_ssm shape mismatch")
    _require(tuple(C_ssm.shape) == (bsz, L, n), "C_ssm shape mismatch")
    _require(tuple(D_ssm.shape) == (dm,), "D_ssm shape mismatch")
    devs = {t.device for _, t in named}
    _require(len(devs) == 1, "all inputs must be on the same device")
    if h_prev is not None:
        if require_device:
            _require(h_prev.is_cuda, "h_prev must be a CUDA tensor")
        _require(h_prev.dtype == u.dtype, "h_prev dtype must match u dtype")
        _require(h_prev.dim() == 0 or h_prev.stride(-1) == 1 or h_prev.size(-1) == 1,
                 "h_prev must be contiguous in the last dimension")
        _require(h_prev.dim() == 3, "h_prev must be 3D (batch, dim, state)")
        _require(tuple(h_prev.shape) == (bsz, dm, n), "h_prev shape must be (B, D, N)")
        _require(h_prev.device == u.device, "h_prev must be on the same device as u")


@functools.lru_cache(maxsize=1024)
def ckpt_count(seqlen: int) -> int:
    return int(_lib.lib().mwc_ssm_ckpt_count(seqlen))


# The launch plan (and so the workspace size) depends on the shape and on the MWC_NSEG / MWC_CFOLD /
# MWC_SPL overrides, which the library reads at call time: the sizes are cached under both.
_PLAN_ENV = ("MWC_NSEG", "MWC_CFOLD", "MWC_SPL")


@functools.lru_cache(maxsize=1024)
def _workspace_bytes(which: str, bsz: int, L: int, dm: int, n: int, env: tuple) -> int:
    fn = _lib.lib().mwc_ssm_fwd_workspace_size if which == "fwd" else _lib.lib().mwc_ssm_bwd_workspace_size
    return int(fn(bsz, L, dm, n))


def workspace_bytes(which: str, bsz: int, L: int, dm: int, n: int) -> int:
    return _workspace_bytes(which, bsz, L, dm, n, tuple(os.environ.get(k) for k in _PLAN_ENV))


def check_transforms(u, delta_bias=None, z=None):
    """The optional elementwise transforms around the scan: delta_bias (D,), z (B, L, D)."""
    bsz, L, dm = u.shape
    for name, t, shape in (("delta_bias", delta_bias, (dm,)), ("z", z, (bsz, L, dm))):
        if t is None:
            continue
        if t.device != u.device:
            raise RuntimeError(f"{name} must be on the same device as u")
        if t.dtype != u.dtype:
            raise RuntimeError(f"{name} dtype must match u dtype")
        if tuple(t.shape) != shape:
            raise RuntimeError(f"{name} shape must be {shape}")


def ssm_forward_xf(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, *, delta_bias=None, delta_softplus=False,
                   z=None, want_out=True, want_ungated=False, want_h_last=True, want_ckpt=False):
    """Fused forward with the optional transforms (delta' = softplus(delta + delta_bias),
    out_z = out * silu(z)). Returns (out_z or out, ungated out or None, h_last or None, ckpt or None).

    ckpt is fp32 (B, ceil(L/16), D, N): the state before every 16th step,
    which the backward restarts from."""
    check_ssm_inputs(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev)
    check_transforms(u, delta_bias, z)
    u, delta, A, B_ssm, C_ssm, D_ssm = (t.contiguous() for t in (u, delta, A, B_ssm, C_ssm, D_ssm))
    h_prev = None if h_prev is None else h_prev.contiguous()
    delta_bias = None if delta_bias is None else delta_bias.contiguous()
    z = None if z is None else z.contiguous()
    L_ = _lib.lib()
    bsz, L, dm = u.shape
    n = A.size(1)
    dev = u.device
    gated = z is not None
    out = torch.empty_like(u) if (want_out and not gated) or (gated and want_ungated) else None
    out_z = torch.empty_like(u) if gated and want_out else None
    h_last = torch.empty(bsz, dm, n, dtype=u.dtype, device=dev) if want_h_last else None
    ckpt = (torch.empty(bsz, ckpt_count(L), dm, n, dtype=torch.float32, device=dev)
            if want_ckpt else None)
    nbytes = workspace_bytes("fwd", bsz, L, dm, n)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)
    with _on_device(dev):
        st = L_.mwc_ssm_fwd_ex(_dtype_code(u), _ptr(u), _ptr(delta), _ptr(A), _ptr(B_ssm), _ptr(C_ssm),
                               _ptr(D_ssm), _ptr(h_prev), _ptr(delta_bias), int(bool(delta_softplus)), _ptr(z),
                               _ptr(out), _ptr(out_z), _ptr(h_last), _ptr(ckpt), bsz, L, dm, n,
                               ws.data_ptr(), nbytes, _stream(dev))
    _lib.check(st, "mwc_ssm_fwd_ex")
    return (out_z if gated else out), (out if gated else None), h_last, ckpt


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
    (du, ddelta, dA, dB, dC, dD, dh_prev or None, ddelta_bias or None, dz or None), in u's dtype."""
    u, delta, A, B_ssm, C_ssm, D_ssm = (t.contiguous() for t in (u, delta, A, B_ssm, C_ssm, D_ssm))
    bsz, L, dm = u.shape
    n = A.size(1)
    _require(n in NSTATES, "Only N=16 (or 8, 32, 64) is supported")
    dout = dout.to(u.dtype).contiguous()
    _require(tuple(dout.shape) == (bsz, L, dm), "dout shape mismatch")
    if dh_last is not None:
        dh_last = dh_last.to(u.dtype).contiguous()
        _require(tuple(dh_last.shape) == (bsz, dm, n), "dh_last shape must be (B, D, N)")
    _require(ckpt is not None and ckpt.dtype == torch.float32 and ckpt.is_contiguous()
             and tuple(ckpt.shape) == (bsz, ckpt_count(L), dm, n), "ckpt does not match the inputs")
    check_transforms(u, delta_bias, z)
    delta_bias = None if delta_bias is None else delta_bias.contiguous()
    if z is not None:
        z = z.contiguous()
        _require(out_ungated is not None and tuple(out_ungated.shape) == (bsz, L, dm),
                 "the ungated forward output is needed with z")
        out_ungated = out_ungated.to(u.dtype).contiguous()
    L_ = _lib.lib()
    dev = u.device
    du = torch.empty_like(u)
    ddelta = torch.empty_like(u)
    dA = torch.empty_like(A)
    dB = torch.empty_like(B_ssm)
    dC = torch.empty_like(C_ssm)
    dD = torch.empty_like(D_ssm)
    dh_prev = torch.empty(bsz, dm, n, dtype=u.dtype, device=dev) if want_dh_prev else None
    dbias = torch.empty_like(delta_bias) if delta_bias is not None else None
    dz = torch.empty_like(z) if z is not None else None
    nbytes = workspace_bytes("bwd", bsz, L, dm, n)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)
    with _on_device(dev):
        st = L_.mwc_ssm_bwd_ex(_dtype_code(u), _ptr(u), _ptr(delta), _ptr(A), _ptr(B_ssm), _ptr(C_ssm),
                               _ptr(D_ssm), None, _ptr(delta_bias), int(bool(delta_softplus)), _ptr(z),
                               _ptr(out_ungated if z is not None else None), _ptr(dout), _ptr(dh_last), _ptr(ckpt),
                               _ptr(du), _ptr(ddelta), _ptr(dA), _ptr(dB), _ptr(dC), _ptr(dD), _ptr(dbias),
                               _ptr(dz), _ptr(dh_prev), bsz, L, dm, n, ws.data_ptr(), nbytes, _stream(dev))
    _lib.check(st, "mwc_ssm_bwd_ex")
    return du, ddelta, dA, dB, dC, dD, dh_prev, dbias, dz


def ssm_backward(u, delta, A, B_ssm, C_ssm, D_ssm, dout, ckpt, dh_last=None, want_dh_prev=False):
    """Fused backward. Returns (du, ddelta, dA, dB, dC, dD, dh_prev or None), in u's dtype."""
    return ssm_backward_xf(u, delta, A, B_ssm, C_ssm, D_ssm, dout, ckpt, dh_last, want_dh_prev)[:7]


def ssm_step(u, delta, A, B_ssm, C_ssm, D_ssm, h, *, delta_bias=None, delta_softplus=False, z=None,
             out_state=None):
    """One decode step: u, delta, z (B, D); A (D, N); B_ssm, C_ssm (B, N); D_ssm (D,); h (B, D, N).
    Returns (out (B, D) -- gated by silu(z) when z is given --, h_new (B, D, N)). out_state, when
    given, receives h_new and may be h itself (in-place update)."""
    named = (("u", u), ("delta", delta), ("A", A), ("B_ssm", B_ssm), ("C_ssm", C_ssm), ("D_ssm", D_ssm), ("h", h))
    for name, t in named:
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be a CUDA tensor")
        if t.dtype != u.dtype:
            raise RuntimeError(f"{name} dtype must match u dtype")
    _require(u.dtype in STORAGE_DTYPES, "u must be float32/float16 (or bfloat16)")
    _require(u.dim() == 2, "u must be 2D (batch, dim) for a step")
    bsz, dm = u.shape
    _require(A.dim() == 2 and A.size(1) in NSTATES, "Only N=16 (or 8, 32, 64) is supported")
    n = A.size(1)
    for name, t, shape in (("delta", delta, (bsz, dm)), ("A", A, (dm, n)), ("B_ssm", B_ssm, (bsz, n)),
                           ("C_ssm", C_ssm, (bsz, n)), ("D_ssm", D_ssm, (dm,)), ("h", h, (bsz, dm, n)),
                           ("delta_bias", delta_bias, (dm,)), ("z", z, (bsz, dm))):
        if t is not None:
            if tuple(t.shape) != shape:
                raise RuntimeError(f"{name} shape must be {shape}")
            if t.dtype != u.dtype or t.device != u.device:
                raise RuntimeError(f"{name} must match u's dtype and device")
    align = 16  # the kernel moves a lane's states as one 16-byte vector

    def aligned(t):
        t = t.contiguous()
        return t if t.data_ptr() % align == 0 else t.clone()

    u, delta, D_ssm = (t.contiguous() for t in (u, delta, D_ssm))
    A, B_ssm, C_ssm, h = (aligned(t) for t in (A, B_ssm, C_ssm, h))
    delta_bias = None if delta_bias is None else delta_bias.contiguous()
    z = None if z is None else z.contiguous()
    if out_state is None:
        out_state = torch.empty_like(h)
    _require(out_state.is_contiguous() and tuple(out_state.shape) == (bsz, dm, n) and out_state.dtype == u.dtype
             and out_state.data_ptr() % align == 0,
             "out_state must be a contiguous, 16-byte-aligned (B, D, N) tensor of u's dtype")
    out = torch.empty_like(u)
    L_ = _lib.lib()
    with _on_device(u.device):
        st = L_.mwc_ssm_step(_dtype_code(u), _ptr(u), _ptr(delta), _ptr(A), _ptr(B_ssm), _ptr(C_ssm), _ptr(D_ssm),
                             _ptr(h), _ptr(delta_bias), int(bool(delta_softplus)), _ptr(z),
                             None if z is not None else _ptr(out), _ptr(out) if z is not None else None,
                             _ptr(out_state), bsz, dm, n, _stream(u.device))
    _lib.check(st, "mwc_ssm_step")
    return out, out_state


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
