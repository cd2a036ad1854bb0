"""GPU parity of parallel_scan_fn (forward and adjoint) against the float64 oracle."""
import numpy as np
import pytest
import torch

from mamba_windows_cuda import parallel_scan_fn, parallel_scan_ref, workloads
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.float16: dict(rtol=1e-2, atol=1e-2),
       torch.bfloat16: dict(rtol=2e-2, atol=2e-2)}


def _np(t):
    return t.detach().cpu().double().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 32, 128, 16), (1, 16, 64, 8), (3, 5, 1000, 3), (2, 1, 1, 7),
                                   (2, 777, 40), (1, 300, 1024), (2, 129, 64)])
def test_pscan_forward_backward(dev, shape, dtype):
    print(f"case pscan shape={shape} dtype={dtype}", flush=True)
    g = torch.Generator().manual_seed(len(shape) * 100 + shape[-2])
    A = (0.5 + 0.5 * torch.rand(shape, generator=g)).to(dtype)
    X = torch.randn(shape, generator=g).to(dtype)
    dH = torch.randn(shape, generator=g).to(dtype)
    Ad = A.to(dev).requires_grad_(True)
    Xd = X.to(dev).requires_grad_(True)
    H = parallel_scan_fn(Ad, Xd)
    H.backward(dH.to(dev))
    torch.cuda.synchronize()
    ref = orc.pscan_fwd(A, X)
    np.testing.assert_allclose(_np(H), ref, **TOL[dtype])
    # adjoint with the oracle's own H (the kernel's H differs only by rounding)
    rdA, rdX = orc.pscan_bwd(A, torch.from_numpy(ref), dH)
    np.testing.assert_allclose(_np(Xd.grad), rdX, **TOL[dtype])
    np.testing.assert_allclose(_np(Ad.grad), rdA, **TOL[dtype])


def test_pscan_matches_reference_loop_and_ignores_A0(dev):
    """parallel_scan_ref semantics (pscan.py:153-171): H_0 = X_0 whatever A_0 is."""
    g = torch.Generator().manual_seed(2)
    A = torch.rand(2, 3, 50, 4, generator=g)
    X = torch.randn(2, 3, 50, 4, generator=g)
    H = parallel_scan_fn(A.to(dev), X.to(dev)).cpu()
    torch.testing.assert_close(H, parallel_scan_ref(A, X), rtol=1e-5, atol=1e-5)
    A2 = A.clone()
    A2[:, :, 0] = 77.0
    assert torch.equal(parallel_scan_fn(A2.to(dev), X.to(dev)).cpu(), H)


def test_pscan_config4b(dev):
    """(4, 65536, 1024) fp32 with a ~ U(0.9, 1), b ~ N(0, 1), against the float64 scan."""
    a, b = workloads.pscan_inputs()
    H = parallel_scan_fn(a.to(dev), b.to(dev))
    torch.cuda.synchronize()
    ref = orc.pscan_fwd(a, b)
    np.testing.assert_allclose(_np(H), ref, rtol=1e-3, atol=1e-4)


def test_scan_beyond_2_31_elements(dev):
    """(4, 2^20, 1024) fp32, 2^32 elements per tensor (the last sequence starts 3*2^30 elements in, its
    look-back chains are 8192 tiles long): the forward and the adjoint address with 64-bit offsets.
    Checked by restarting the scan: the last 4096 steps of the last sequence equal a scan of those
    steps whose first input folds in the state before them, and the adjoint's last steps equal the
    adjoint of that shorter scan (it depends only on later steps)."""
    from mamba_windows_cuda.pscan import pscan_check

    S, L, C, T = 4, 1 << 20, 1024, 4096
    print(f"case scan beyond 2^31 elements ({S}, {L}, {C})", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    A = torch.rand(S, L, C, generator=g, device=dev).mul_(0.1).add_(0.9).requires_grad_(True)
    X = torch.randn(S, L, C, generator=g, device=dev).requires_grad_(True)
    H = parallel_scan_fn(A, X)
    dH = torch.randn(S, L, C, generator=g, device=dev)
    H.backward(dH)
    t0 = L - T
    with torch.no_grad():
        At = A[S - 1:, t0:].clone()
        Xt = X[S - 1:, t0:].clone()
        Xt[:, 0] += At[:, 0] * H[S - 1:, t0 - 1]
    At.requires_grad_(True)
    Xt.requires_grad_(True)
    Ht = parallel_scan_fn(At, Xt)
    Ht.backward(dH[S - 1:, t0:])
    pscan_check()
    torch.cuda.synchronize()
    torch.testing.assert_close(H[S - 1:, t0:], Ht, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(X.grad[S - 1:, t0:], Xt.grad, rtol=1e-4, atol=1e-4)
    # dA_t = g_t * H_{t-1}: the restarted scan's first step has no H_{t-1} of its own
    torch.testing.assert_close(A.grad[S - 1:, t0 + 1:], At.grad[:, 1:], rtol=1e-4, atol=1e-4)
    del A, X, H, dH
    torch.cuda.empty_cache()  # hand the ~100 GB back before the next test
