"""TEST INFRASTRUCTURE ONLY: numpy front-end of the float64 C oracle.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker. The product path never does.

Each function restates one reference function (file:line in
/root/reference, zouyuanqing/mamba-windows-cuda):

* ``ssm_fwd``   -- ``selective_scan_ref`` (mamba_windows_cuda/mamba_cuda.py:875-946)
* ``ssm_bwd``   -- autograd through ``selective_scan_ref`` (tests/test_selective_scan.py:361-364)
* ``pscan_fwd`` -- ``parallel_scan_ref`` (mamba_windows_cuda/pscan.py:153-171)
* ``pscan_bwd`` -- the adjoint of ``parallel_scan_ref``
* ``ssm_fwd_xf`` / ``ssm_bwd_xf`` -- ``ssm_fwd`` / ``ssm_bwd`` composed with the elementwise
  transforms a Mamba block applies around the scan (delta' = softplus(delta + delta_bias),
  out_z = out * silu(z)); the reference has no counterpart (it rejects them), so these follow the
  textbook definitions, and the chain rule is written out here in float64

All arithmetic is float64 on the (dtype-rounded) inputs. Pins live in
tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_ssm.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the C oracle with gcc (via the Makefile next to this file)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s"] + (["-B"] if force else []) + ["-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        lib.oracle_ssm_fwd.argtypes = [I, I, I, I, P, P, P, P, P, P, P, ctypes.c_int, P, P]
        lib.oracle_ssm_bwd.argtypes = [I, I, I, I, P, P, P, P, P, P, P, P, P, ctypes.c_int,
                                       P, P, P, P, P, P, P, P, P, P]
        lib.oracle_pscan_fwd.argtypes = [I, I, I, P, P, P]
        lib.oracle_pscan_bwd.argtypes = [I, I, I, P, P, P, P, P]
        for f in (lib.oracle_ssm_fwd, lib.oracle_ssm_bwd, lib.oracle_pscan_fwd, lib.oracle_pscan_bwd):
            f.restype = None
        _lib = lib
    return _lib


def _f64(x):
    """float64 C-contiguous numpy copy of a numpy array or torch tensor (None passes)."""
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().to("cpu")
        import torch

        x = x.to(torch.float64).numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=np.float64))


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def ssm_fwd(u, delta, A, B, C, D, h_prev=None, clamp=False):
    """Returns (out (B,L,D), h_last (B,D,N)) in float64."""
    u, delta, A, B, C, D, h_prev = map(_f64, (u, delta, A, B, C, D, h_prev))
    Bsz, L, Dm = u.shape
    N = A.shape[1]
    out = np.empty((Bsz, L, Dm))
    h_last = np.empty((Bsz, Dm, N))
    _load().oracle_ssm_fwd(Bsz, L, Dm, N, _p(u), _p(delta), _p(A), _p(B), _p(C), _p(D),
                           _p(h_prev), int(bool(clamp)), _p(out), _p(h_last))
    return out, h_last


def ssm_bwd(u, delta, A, B, C, D, dout, h_prev=None, dh_last=None, clamp=False):
    """Returns dict du, ddelta, dA, dB, dC, dD, dh_prev (all float64), plus conditioning measures for
    tests (not gradients): the running-error magnitudes dA_abs (D,N), ddelta_abs and du_abs (B,L,D) --
    each output's sum with every term replaced by its magnitude and the state h and adjoint
    g = dL/dh_t by recurrences run on magnitudes (H_t = dA_t H_{t-1} + |delta u B|, H_{-1} = |h_prev|;
    G_t = |dout_t C_t| + dA_{t+1} G_{t+1}, G_{L-1} including |dh_last|):
    dA_abs = sum_{b,t} |delta| G dA_t H_{t-1}, ddelta_abs = sum_n |A| G dA_t H_{t-1} + |u| sum_n G |B|,
    du_abs = |D dout| + |delta| sum_n G |B| -- and dD_abs = sum_{b,t} |dout u| (D,). An fp32 evaluation
    of an output errs by a few eps32 times its magnitude sum, whatever cancels in h, g or the sum."""
    u, delta, A, B, C, D, dout, h_prev, dh_last = map(
        _f64, (u, delta, A, B, C, D, dout, h_prev, dh_last))
    Bsz, L, Dm = u.shape
    N = A.shape[1]
    r = dict(du=np.empty((Bsz, L, Dm)), ddelta=np.empty((Bsz, L, Dm)), dA=np.empty((Dm, N)),
             dB=np.empty((Bsz, L, N)), dC=np.empty((Bsz, L, N)), dD=np.empty((Dm,)),
             dh_prev=np.empty((Bsz, Dm, N)), dA_abs=np.empty((Dm, N)), ddelta_abs=np.empty((Bsz, L, Dm)),
             du_abs=np.empty((Bsz, L, Dm)))
    _load().oracle_ssm_bwd(Bsz, L, Dm, N, _p(u), _p(delta), _p(A), _p(B), _p(C), _p(D),
                           _p(h_prev), _p(dout), _p(dh_last), int(bool(clamp)),
                           _p(r["du"]), _p(r["ddelta"]), _p(r["dA"]), _p(r["dB"]), _p(r["dC"]),
                           _p(r["dD"]), _p(r["dh_prev"]), _p(r["dA_abs"]), _p(r["ddelta_abs"]),
                           _p(r["du_abs"]))
    r["dD_abs"] = np.abs(dout * u).sum(axis=(0, 1))
    return r


def _softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _delta_xf(delta, delta_bias, delta_softplus):
    d = _f64(delta)
    if delta_bias is not None:
        d = d + _f64(delta_bias)[None, None, :]
    return _softplus(d) if delta_softplus else d, d


def ssm_fwd_xf(u, delta, A, B, C, D, h_prev=None, delta_bias=None, delta_softplus=False, z=None, clamp=False):
    """Returns (out_z or out, h_last, ungated out) in float64."""
    dxf, _ = _delta_xf(delta, delta_bias, delta_softplus)
    out, h_last = ssm_fwd(u, dxf, A, B, C, D, h_prev, clamp)
    if z is None:
        return out, h_last, out
    zz = _f64(z)
    return out * zz * _sigmoid(zz), h_last, out


def ssm_bwd_xf(u, delta, A, B, C, D, dout, h_prev=None, dh_last=None, delta_bias=None, delta_softplus=False,
               z=None, clamp=False):
    """ssm_bwd through the transforms. Returns the ssm_bwd dict (ddelta and ddelta_abs w.r.t. the raw
    delta) plus 'ddelta_bias', its magnitude sum 'ddelta_bias_abs' = sum_{b,t} ddelta_abs, and 'dz'
    (None when the transform is absent)."""
    dxf, dpre = _delta_xf(delta, delta_bias, delta_softplus)
    g = _f64(dout)
    dz = None
    if z is not None:
        zz = _f64(z)
        sz = _sigmoid(zz)
        y, _ = ssm_fwd(u, dxf, A, B, C, D, h_prev, clamp)
        dz = g * y * sz * (1.0 + zz * (1.0 - sz))
        g = g * zz * sz
    r = ssm_bwd(u, dxf, A, B, C, D, g, h_prev, dh_last, clamp)
    if delta_softplus:
        r["ddelta"] = r["ddelta"] * _sigmoid(dpre)
        r["ddelta_abs"] = r["ddelta_abs"] * _sigmoid(dpre)
    r["ddelta_bias"] = r["ddelta"].sum(axis=(0, 1)) if delta_bias is not None else None
    r["ddelta_bias_abs"] = r["ddelta_abs"].sum(axis=(0, 1)) if delta_bias is not None else None
    r["dz"] = dz
    return r


def _as3(x):
    """View (B, D, L, N) as (B*D, L, N); 3-D inputs pass through."""
    if x.ndim == 4:
        b, d, l, n = x.shape
        return x.reshape(b * d, l, n)
    if x.ndim == 3:
        return x
    raise ValueError("parallel scan inputs must be 3-D or 4-D")


def pscan_fwd(A, X):
    """H with H_0 = X_0, H_t = A_t H_{t-1} + X_t along axis -2 (float64, input shape)."""
    A, X = _f64(A), _f64(X)
    shape = X.shape
    a3, x3 = _as3(A), _as3(X)
    H = np.empty_like(x3)
    _load().oracle_pscan_fwd(x3.shape[0], x3.shape[1], x3.shape[2], _p(a3), _p(x3), _p(H))
    return H.reshape(shape)


def pscan_bwd(A, H, dH):
    """Returns (dA, dX) for H = pscan_fwd(A, X) and upstream gradient dH."""
    A, H, dH = _f64(A), _f64(H), _f64(dH)
    shape = H.shape
    a3, h3, g3 = _as3(A), _as3(H), _as3(dH)
    dA = np.empty_like(h3)
    dX = np.empty_like(h3)
    _load().oracle_pscan_bwd(h3.shape[0], h3.shape[1], h3.shape[2], _p(a3), _p(h3), _p(g3),
                             _p(dA), _p(dX))
    return dA.reshape(shape), dX.reshape(shape)
