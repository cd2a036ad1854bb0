"""Selective scan (Mamba-1, N=16; also N=8, 32, 64) on MI355X -- the drop-in for
``mamba_windows_cuda.mamba_cuda`` of zouyuanqing/mamba-windows-cuda.

Same public names, signatures, shapes and dtype rules as the reference
(mamba_windows_cuda/mamba_cuda.py:1044-1219); the work runs in the gfx950
kernels of libmwc_ssm.so, called through the PyTorch operators of libmwc_torch.so
(csrc/torch_ops.cpp). Differences from the
reference, all in the direction of correctness:

* one fused forward and one fused backward serve every mode. The stateful
  path no longer runs a Python loop over L in the forward (reference 1065-1068)
  or the backward (987-1025), and its gradients are the true adjoint (the
  reference's hand-written backward, 949-1041, mis-scales dA and ddelta);
* h_prev/h_last are honoured by the backward as well (the reference's CUDA
  backward kernels start from h = 0), giving dh_prev when h_prev is given;
* nothing is saved for backward when no input requires grad.

Checkpoint levels (the memory/speed knob of FusedSelectiveScan,
selective_scan_cuda_ext.py:573-621, also accepted by SelectiveScanCuda):
0 = the forward stores the fp32 state every 16 steps (B*ceil(L/16)*D*N*4
bytes) and the backward restarts from it; 1 = only the inputs are kept and
the backward first re-runs a state-only forward pass to rebuild them.
"""
from __future__ import annotations

import torch

from . import _lib, ops

_scan_op = None
_step_op = None  # torch.ops.mwc.ssm_step: the decode step's checks and launch in C++


def _ssm_scan(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, checkpoint_lvl, z, delta_bias, delta_softplus):
    """(out, h_last) through ``torch.ops.mwc.ssm_scan`` (csrc/torch_ops.cpp): the same checks,
    kernels and gradients as SelectiveScanCudaFunction, with the argument checks, allocation,
    launch and autograd Function in C++ rather than Python."""
    global _scan_op
    if _scan_op is None:
        _scan_op = _lib.torch_ops().ssm_scan.default
    return _scan_op(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, checkpoint_lvl, z, delta_bias, bool(delta_softplus))


def _forward_impl(ctx, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, checkpoint_lvl, z=None, delta_bias=None,
                  delta_softplus=False):
    if checkpoint_lvl not in (0, 1):
        raise RuntimeError(f"checkpoint_lvl must be 0 or 1 (got {checkpoint_lvl})")
    grads_of = list(ctx.needs_input_grad[:6]) + [h_prev is not None and ctx.needs_input_grad[6]]
    if len(ctx.needs_input_grad) > 8:  # the transform arguments (z, delta_bias)
        grads_of += [z is not None and ctx.needs_input_grad[8], delta_bias is not None and ctx.needs_input_grad[9]]
    need_grad = any(grads_of)
    out, out_ungated, h_last, ckpt = ops.ssm_forward_xf(
        u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, delta_bias=delta_bias, delta_softplus=delta_softplus, z=z,
        want_ungated=need_grad and z is not None, want_ckpt=need_grad and checkpoint_lvl == 0)
    ctx.has_h_prev = h_prev is not None
    ctx.need_grad = need_grad
    ctx.delta_softplus = bool(delta_softplus)
    if need_grad:
        ctx.save_for_backward(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, ckpt, z, delta_bias, out_ungated)
    ctx.set_materialize_grads(False)
    return out, h_last


def _backward_impl(ctx, dout, dh_last):
    u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, ckpt, z, delta_bias, out_ungated = ctx.saved_tensors
    xf = dict(delta_bias=delta_bias, delta_softplus=ctx.delta_softplus, z=z)
    if ckpt is None:  # recompute level: rebuild the state checkpoints (and the ungated output for dz)
        _, out_ungated, _, ckpt = ops.ssm_forward_xf(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, want_out=False,
                                                     want_ungated=z is not None, want_h_last=False,
                                                     want_ckpt=True, **xf)
    if dout is None:
        dout = torch.zeros_like(u)
    want_dh_prev = ctx.has_h_prev and ctx.needs_input_grad[6]
    return ops.ssm_backward_xf(u, delta, A, B_ssm, C_ssm, D_ssm, dout, ckpt, dh_last, want_dh_prev=want_dh_prev,
                               out_ungated=out_ungated, **xf)


class SelectiveScanCudaFunction(torch.autograd.Function):
    """(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, checkpoint_lvl=0, z=None, delta_bias=None,
    delta_softplus=False) -> (out, h_last); backward returns dh_prev when h_prev is given
    (mamba_cuda.py:1044-1096). The last three arguments are the fused transforms (delta' =
    softplus(delta + delta_bias), out = scan * silu(z)); the reference has no counterpart.
    A Python autograd Function over the raw operators (ops.ssm_forward_xf / ssm_backward_xf);
    SelectiveScanCuda and FusedSelectiveScan call ``torch.ops.mwc.ssm_scan``, whose autograd
    Function is C++, with bitwise the same results and less host time per call."""

    @staticmethod
    def forward(ctx, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, checkpoint_lvl=0, z=None, delta_bias=None,
                delta_softplus=False):
        return _forward_impl(ctx, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, checkpoint_lvl, z, delta_bias,
                             delta_softplus)

    @staticmethod
    def backward(ctx, dout, dh_last):
        du, ddelta, dA, dB, dC, dD, dh_prev, dbias, dz = _backward_impl(ctx, dout, dh_last)
        return du, ddelta, dA, dB, dC, dD, dh_prev, None, dz, dbias, None


class SelectiveScanFn(torch.autograd.Function):
    """Recompute level (the reference's V1, mamba_cuda.py:1099-1133): saves only the inputs."""

    @staticmethod
    def forward(ctx, u, delta, A, B_ssm, C_ssm, D_ssm):
        out, _ = _forward_impl(ctx, u, delta, A, B_ssm, C_ssm, D_ssm, None, 1)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        return tuple(_backward_impl(ctx, grad_out, None)[:6])


class SelectiveScanFnV2(torch.autograd.Function):
    """Save level (the reference's V2, mamba_cuda.py:1136-1169): the forward keeps state checkpoints."""

    @staticmethod
    def forward(ctx, u, delta, A, B_ssm, C_ssm, D_ssm):
        out, _ = _forward_impl(ctx, u, delta, A, B_ssm, C_ssm, D_ssm, None, 0)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        return tuple(_backward_impl(ctx, grad_out, None)[:6])


class SelectiveScanCuda(torch.nn.Module):
    """Mamba selective scan on MI355X with autograd (mamba_cuda.py:1172-1219).

    ``forward(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None) -> out`` and
    ``forward_with_state(...) -> (out, h_last)``. Shapes: u, delta (B, L, D);
    A (D, N); B_ssm, C_ssm (B, L, N); D_ssm (D,); h_prev, h_last (B, D, N), with
    N = 16 as in the reference, or 8, 32, 64. All tensors fp32 or all fp16 (or
    all bf16), on the GPU; outputs and gradients take the
    input dtype. ``checkpoint_lvl`` (keyword, default 0) picks the memory/speed
    trade-off described in the module docstring. The calls go through the C++ operator
    ``torch.ops.mwc.ssm_scan`` (argument checks, allocation, launch and the autograd Function
    in C++).

    Keyword-only extras fused into the kernels (not in the reference; the
    options a Mamba block applies around the scan): ``delta_bias`` (D,) and
    ``delta_softplus`` give delta' = softplus(delta + delta_bias); ``z``
    (B, L, D) gates the output, out * silu(z). Gradients flow to z and
    delta_bias.
    """

    def __init__(self, checkpoint_lvl: int = 0):
        super().__init__()
        self.checkpoint_lvl = checkpoint_lvl

    def forward(self, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, *, z=None, delta_bias=None,
                delta_softplus=False):
        return _ssm_scan(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, self.checkpoint_lvl, z, delta_bias,
                         delta_softplus)[0]

    def forward_with_state(self, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, *, z=None, delta_bias=None,
                           delta_softplus=False):
        """Returns (out (B, L, D), h_last (B, D, N)); h_last feeds the next chunk's h_prev."""
        return _ssm_scan(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, self.checkpoint_lvl, z, delta_bias,
                         delta_softplus)

    def step(self, u, delta, A, B_ssm, C_ssm, D_ssm, h, *, z=None, delta_bias=None, delta_softplus=False,
             out_state=None):
        """One decode step (inference only; not in the reference, whose way to advance one token is
        forward_with_state with L=1). u, delta, z: (B, D); B_ssm, C_ssm: (B, N); h: (B, D, N).
        Returns (out (B, D), h_new (B, D, N)); pass out_state=h to update the state in place."""
        global _step_op
        if _step_op is None:
            _step_op = _lib.torch_ops().ssm_step.default
        return _step_op(u, delta, A, B_ssm, C_ssm, D_ssm, h, z, delta_bias, bool(delta_softplus), out_state)


def selective_scan_ref(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, return_intermediates=False):
    """Plain-PyTorch sequential selective scan (any device, autograd-capable),
    the reference's ``selective_scan_ref`` API (mamba_cuda.py:875-946).

    Returns (out (B,L,D), h_last (B,D,N)) and, with return_intermediates, a
    dict of the (B,D,N,L) tensors 'h_states', 'dA', 'dBu' plus the transposed
    inputs and, beyond the reference's keys, 'A' (which the adjoint of delta
    needs; see selective_scan_backward). Not used by the GPU path.
    """
    bsz, L, dm = u.shape
    n = A.shape[1]
    u_t, d_t = u.transpose(1, 2), delta.transpose(1, 2)
    B_t, C_t = B_ssm.transpose(1, 2), C_ssm.transpose(1, 2)
    if h_prev is None:
        h_prev = torch.zeros(bsz, dm, n, device=u.device, dtype=u.dtype)
    dA = torch.exp(d_t.unsqueeze(2) * A.unsqueeze(0).unsqueeze(-1))   # (B,D,N,L)
    dBu = (d_t * u_t).unsqueeze(2) * B_t.unsqueeze(1)                # (B,D,N,L)
    h = h_prev
    states = []
    for t in range(L):
        h = dA[..., t] * h + dBu[..., t]
        states.append(h)
    h_states = torch.stack(states, dim=-1) if states else h_prev.new_zeros(bsz, dm, n, 0)
    y = (C_t.unsqueeze(1) * h_states).sum(2) + u_t * D_ssm.view(1, -1, 1)
    out = y.transpose(1, 2)
    if return_intermediates:
        return out, h, {"h_states": h_states, "dA": dA, "dBu": dBu, "u_t": u_t, "delta_t": d_t,
                        "B_t": B_t, "C_t": C_t, "h_prev": h_prev, "A": A}
    return out, h


def recover_A(dA, delta_t):
    """A (D, N) from the reference intermediates' decay factors dA = exp(delta*A) (B, D, N, L) and
    delta_t (B, D, L): A = log(dA) / delta at, for each (d, n), the (b, t) with the largest delta
    whose factor is a normal number (log(dA) then carries an absolute error of about one ulp of 1,
    so A's absolute error is about eps / delta: 7e-7 at delta = 0.09 in fp32). Raises
    RuntimeError for a (d, n) with no usable step (delta = 0 everywhere, where the decay factors do
    not depend on A, or every factor underflowed); pass A explicitly then."""
    bsz, dm, n, L = dA.shape
    dl = delta_t.unsqueeze(2).expand(bsz, dm, n, L)
    usable = (dl > 0) & (dA >= torch.finfo(dA.dtype).tiny) & torch.isfinite(dA)
    score = torch.where(usable, dl, torch.full_like(dl, -1.0))
    score = score.permute(1, 2, 0, 3).reshape(dm, n, bsz * L)
    best = score.argmax(-1, keepdim=True)
    if not bool((score.gather(-1, best) > 0).all()):
        raise RuntimeError("selective_scan_backward: A cannot be recovered from intermediates['dA'] for every "
                           "(d, n) (delta is 0 or the decay factors underflow); pass A=")
    pick = lambda x: x.permute(1, 2, 0, 3).reshape(dm, n, bsz * L).gather(-1, best).squeeze(-1)
    return torch.log(pick(dA)) / pick(dl)


def selective_scan_backward(dout, dh_last, intermediates, D_ssm, A=None):
    """Gradients of the selective scan from ``selective_scan_ref``'s intermediates: the reference
    API (mamba_cuda.py:949-1041), same arguments and return order
    ``(du, ddelta, dA, dB_ssm, dC_ssm, dD_ssm, dh_prev)``; plain PyTorch on the intermediates'
    device, not used by the GPU path.

    Deliberate difference: this returns the true adjoint (what autograd gives through
    ``selective_scan_ref``). The reference's loop hands du, ddelta and dB the decayed adjoint
    dA_t*g_t where they need g_t (mamba_cuda.py:1012-1025), drops the A*dA_t*h_{t-1} term of
    ddelta, and returns the gradient with respect to the decay factors, sum dh*h_{t-1}
    (1009, 1033), instead of the one with respect to A. Here, with g_t = dout_t*C_t + dA_{t+1}*g_{t+1}
    (g_{L-1} also receives dh_last):
      du = D*dout + delta*sum_n g*B          ddelta = sum_n g*(A*dA_t*h_{t-1} + u*B)
      dA = sum_{b,t} delta*g*dA_t*h_{t-1}    dB = sum_d g*delta*u    dC = sum_d dout*h_t
      dD = sum_{b,t} dout*u                  dh_prev = dA_0*g_0
    The ddelta term needs A itself: it is taken from the ``A`` keyword, else from
    intermediates['A'] (which ``selective_scan_ref`` here adds), else recovered from the reference's
    8-key dict (mamba_cuda.py:934-944) by ``recover_A``. ``dh_last`` may be None (zeros)."""
    h_states, dA_t, u_t, d_t = (intermediates[k] for k in ("h_states", "dA", "u_t", "delta_t"))
    B_t, C_t, h_prev = intermediates["B_t"], intermediates["C_t"], intermediates["h_prev"]
    if A is None:
        A = intermediates["A"] if "A" in intermediates else recover_A(dA_t, d_t)
    A = A.to(h_states.dtype)
    bsz, dm, n, L = h_states.shape
    dout_t = dout.transpose(1, 2).to(h_states.dtype)      # (B, D, L)
    g = (torch.zeros_like(h_prev) if dh_last is None else dh_last.to(h_states.dtype)).clone()
    du_t = torch.empty_like(u_t)
    dd_t = torch.empty_like(d_t)
    dB_t = torch.empty_like(B_t)
    dC_t = torch.empty_like(C_t)
    dA_acc = torch.zeros_like(h_prev)                     # (B, D, N), summed over b at the end
    for t in range(L - 1, -1, -1):
        g = g + dout_t[:, :, t, None] * C_t[:, None, :, t]  # g_t
        prev = h_states[..., t - 1] if t > 0 else h_prev
        s = g * dA_t[..., t] * prev                          # g_t * dA_t * h_{t-1}
        S1 = (g * B_t[:, None, :, t]).sum(-1)                # sum_n g*B
        du_t[:, :, t] = D_ssm * dout_t[:, :, t] + d_t[:, :, t] * S1
        dd_t[:, :, t] = (A * s).sum(-1) + u_t[:, :, t] * S1
        dA_acc = dA_acc + d_t[:, :, t, None] * s
        dB_t[:, :, t] = (g * (d_t[:, :, t] * u_t[:, :, t])[:, :, None]).sum(1)
        dC_t[:, :, t] = (dout_t[:, :, t, None] * h_states[..., t]).sum(1)
        g = g * dA_t[..., t]                                 # carried to t - 1
    dD = (u_t * dout_t).sum(dim=(0, 2))
    return (du_t.transpose(1, 2), dd_t.transpose(1, 2), dA_acc.sum(0), dB_t.transpose(1, 2),
            dC_t.transpose(1, 2), dD, g)
