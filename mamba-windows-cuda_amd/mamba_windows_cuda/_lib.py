"""Loading of the native libraries: the ctypes binding of libmwc_ssm.so, the gfx950 C-ABI library
(include/mwc_ssm.h), and libmwc_torch.so, its PyTorch operators (torch.ops.mwc.*).

This replaces the reference's JIT bootstrap (``_get_selective_scan_cuda_module``,
mamba_windows_cuda/mamba_cuda.py:832-872; ``_get_fused_module``,
selective_scan_cuda_ext.py:530-559): the libraries are built ahead of time with
hipcc and only loaded here. If one is missing its first use fails loudly -- there is
no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# MWC_SSM_LIB: another build of libmwc_ssm.so, used by the ctypes binding and (through its SONAME) by
# the PyTorch operators alike
LIB_PATH = os.environ.get("MWC_SSM_LIB", os.path.join(_HERE, "libmwc_ssm.so"))

MWC_DTYPE_F32 = 0
MWC_DTYPE_F16 = 1
MWC_DTYPE_BF16 = 2
MWC_OK = 0
CKPT_STEPS = 16  # MWC_CKPT_STEPS
NOALLOC_SCRATCH_BYTES = 32 << 20  # MWC_NOALLOC_SCRATCH_BYTES

_lock = threading.RLock()  # torch_ops() loads the C-ABI library under it
_lib = None

P = ctypes.c_void_p
I64 = ctypes.c_int64
SZ = ctypes.c_size_t

_SIGNATURES = {
    "mwc_abi_version": ([], ctypes.c_int),
    "mwc_status_string": ([ctypes.c_int], ctypes.c_char_p),
    "mwc_last_error": ([], ctypes.c_char_p),
    "mwc_ssm_ckpt_count": ([I64], I64),
    "mwc_ssm_fwd_workspace_size": ([I64, I64, I64, I64], SZ),
    "mwc_ssm_fwd": ([ctypes.c_int, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, P, SZ, P], ctypes.c_int),
    # dtype, u, delta, A, B, C, D, h_prev, delta_bias, softplus, z, out, out_z, h_last, ckpt, sizes, ws
    "mwc_ssm_fwd_ex": ([ctypes.c_int, P, P, P, P, P, P, P, P, ctypes.c_int, P, P, P, P, P, I64, I64, I64, I64,
                        P, SZ, P], ctypes.c_int),
    # mwc_ssm_fwd_ex without the workspace arguments (static per-device scratch; allocates nothing)
    "mwc_ssm_fwd_noalloc": ([ctypes.c_int, P, P, P, P, P, P, P, P, ctypes.c_int, P, P, P, P, P, I64, I64, I64,
                             I64, P], ctypes.c_int),
    "mwc_ssm_bwd_workspace_size": ([I64, I64, I64, I64], SZ),
    "mwc_ssm_bwd": ([ctypes.c_int, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, P, SZ, P],
                    ctypes.c_int),
    # dtype, u, delta, A, B, C, D, h_prev, delta_bias, softplus, z, out, dout, dh_last, ckpt,
    # du, ddelta, dA, dB, dC, dD, ddelta_bias, dz, dh_prev, sizes, ws
    "mwc_ssm_bwd_ex": ([ctypes.c_int, P, P, P, P, P, P, P, P, ctypes.c_int, P, P, P, P, P, P, P, P, P, P, P, P, P,
                        P, I64, I64, I64, I64, P, SZ, P], ctypes.c_int),
    # dtype, u, delta, A, B, C, D, h, delta_bias, softplus, z, out, out_z, h_new, batch, dim, dstate, stream
    "mwc_ssm_step": ([ctypes.c_int, P, P, P, P, P, P, P, P, ctypes.c_int, P, P, P, P, I64, I64, I64, P],
                     ctypes.c_int),
    "mwc_pscan_workspace_size": ([I64, I64, I64], SZ),
    "mwc_pscan_fwd": ([ctypes.c_int, P, P, P, I64, I64, I64, P, SZ, P], ctypes.c_int),
    "mwc_pscan_bwd": ([ctypes.c_int, P, P, P, P, P, I64, I64, I64, P, SZ, P], ctypes.c_int),
    # workspace, bytes, nseq, seqlen, ncols, stream
    "mwc_pscan_status": ([P, SZ, I64, I64, I64, P], ctypes.c_int),
    "mwc_pscan_status_async": ([P, SZ, I64, I64, I64, P, P], ctypes.c_int),
}

EXPORTED = tuple(_SIGNATURES)


TORCH_OPS_PATH = os.path.join(_HERE, "libmwc_torch.so")
_torch_ops = None


class NativeLibraryMissing(ImportError):
    pass


def lib():
    """Load (once) and return the native library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryMissing(
                    f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `make -C mamba-windows-cuda_amd/csrc` (hipcc, gfx950)")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = args
                fn.restype = res
            _lib = handle
    return _lib


def torch_ops():
    """Load (once) libmwc_torch.so, the PyTorch operators over the C ABI (csrc/torch_ops.cpp), and
    return their namespace, ``torch.ops.mwc``; raises if it is not built."""
    global _torch_ops
    if _torch_ops is not None:
        return _torch_ops
    with _lock:
        if _torch_ops is None:
            if not os.path.exists(TORCH_OPS_PATH):
                raise NativeLibraryMissing(
                    f"{TORCH_OPS_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `make -C mamba-windows-cuda_amd/csrc`")
            import torch

            # load the C-ABI library first (from LIB_PATH, which MWC_SSM_LIB may point elsewhere): its
            # SONAME then satisfies libmwc_torch.so's dependency, so the operators and the ctypes
            # binding share one copy instead of the RUNPATH one being mapped as well
            lib()
            torch.ops.load_library(TORCH_OPS_PATH)
            _torch_ops = torch.ops.mwc
    return _torch_ops


def check(status: int, what: str) -> None:
    """Raise RuntimeError (the reference's TORCH_CHECK surface) on a non-OK status."""
    if status != MWC_OK:
        L = lib()
        msg = L.mwc_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {L.mwc_status_string(status).decode()}: {msg}")
