"""The reference's own test suite, one test per reference test, run against this package on the GPU.

Each test keeps the reference test's name, shapes, seeds, input distributions, calls and assertions
(mamba_windows_cuda/tests/test_selective_scan.py and test_pscan.py). Three things differ:

* inputs are drawn on the CPU from the same seed and then moved to the GPU (the reference draws
  them on its CUDA device, whose random stream differs), so the values are not the reference's;
* where the reference compares with a torch formula of its own (the cumsum closed form of
  test_selective_scan.py:8-36), this suite compares with the float64 oracle, which the CPU tests
  pin against that closed form; the reference's absolute bound (1e-3) is kept, and the north-star
  tolerances are checked as well;
* test_gradient_flow (test_selective_scan.py:287-330) and test_parallel_scan_gradient
  (test_pscan.py:37-62) build some inputs as `torch.ones(..., requires_grad=True) * 0.01`, which
  is not a leaf, so `.grad` stays None and those assertions cannot hold as written; here the
  scaled tensors are made leaves, which is what the assertions mean.

The 1280^2-step fp16 stream and the long single passes of test_large_shapes_and_streaming
(test_selective_scan.py:195-237) are in tests/test_gpu_api.py (test_long_fp16_stream,
test_long_fp16_single_pass), where they are also checked against a full pass and the oracle.
"""
import numpy as np
import pytest
import torch

from mamba_windows_cuda import SelectiveScanCuda, parallel_scan_fn, parallel_scan_ref, selective_scan_ref
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

# north-star tolerances (|x - y| <= atol + rtol |y|) per storage dtype
TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.float16: dict(rtol=1e-2, atol=1e-2)}


def _inputs(seed, B, L, D, N, dtype, *, delta_val=0.01, h_prev="zeros"):
    """The reference tests' distributions: u, B, C ~ 0.1 N(0,1); delta constant; A = -0.1 U(0,1);
    D_ssm = 0.1; h_prev zeros, N(0,1) or absent. (test_gradient_numerical_accuracy redraws u
    as N(0,1), as the reference test does.)"""
    torch.manual_seed(seed)
    x = dict(u=torch.randn(B, L, D) * 0.1, delta=torch.ones(B, L, D) * delta_val, A=-torch.rand(D, N) * 0.1,
             B=torch.randn(B, L, N) * 0.1, C=torch.randn(B, L, N) * 0.1, D=torch.ones(D) * 0.1)
    if h_prev == "zeros":
        x["h_prev"] = torch.zeros(B, D, N)
    elif h_prev == "randn":
        x["h_prev"] = torch.randn(B, D, N)
    return {k: v.to(dtype) for k, v in x.items()}


def _oracle(x):
    return orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x.get("h_prev"))


def _dev(x, dev):
    return {k: v.to(dev) for k, v in x.items()}


def _maxdiff(got, ref):
    return float(np.abs(got.detach().cpu().double().numpy() - ref).max())


def _args(x):
    return x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"]


@pytest.fixture(scope="module")
def kernel(dev):
    return SelectiveScanCuda().to(dev)


@pytest.mark.parametrize("dtype,seed", [(torch.float16, 0), (torch.float32, 42)], ids=["fp16", "fp32"])
def test_consistency(dev, kernel, dtype, seed):
    """test_consistency_fp16 / test_consistency_fp32 (test_selective_scan.py:46-94)."""
    print(f"case reference consistency {dtype}", flush=True)
    x = _inputs(seed, 1, 1024, 256, 16, dtype)
    g = _dev(x, dev)
    with torch.no_grad():
        out = kernel(*_args(g), g["h_prev"])
    ref, _ = _oracle(x)
    assert np.isfinite(ref).all() and torch.isfinite(out).all()
    assert _maxdiff(out, ref) < 1e-3
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, **TOL[dtype])


def test_nonzero_h_prev(dev, kernel):
    """test_selective_scan.py:96-120: fp16, h_prev ~ N(0,1)."""
    print("case reference nonzero h_prev", flush=True)
    x = _inputs(123, 1, 1024, 256, 16, torch.float16, h_prev="randn")
    g = _dev(x, dev)
    with torch.no_grad():
        out = kernel(*_args(g), g["h_prev"])
    ref, _ = _oracle(x)
    assert torch.isfinite(out).all()
    assert _maxdiff(out, ref) < 1e-3


def test_forward_with_state(dev, kernel):
    """test_selective_scan.py:122-146: out and h_last of forward_with_state."""
    print("case reference forward_with_state", flush=True)
    x = _inputs(456, 1, 1024, 256, 16, torch.float16)
    g = _dev(x, dev)
    with torch.no_grad():
        out, h_last = kernel.forward_with_state(*_args(g), g["h_prev"])
    ref_out, ref_h = _oracle(x)
    assert torch.isfinite(out).all() and torch.isfinite(h_last).all()
    assert _maxdiff(out, ref_out) < 1e-3
    assert _maxdiff(h_last, ref_h) < 1e-3
    np.testing.assert_allclose(h_last.cpu().double().numpy(), ref_h, **TOL[torch.float16])


def test_streaming_consistency(dev, kernel):
    """test_selective_scan.py:148-193: two 1024-step chunks carrying h equal one 2048-step pass."""
    print("case reference streaming consistency", flush=True)
    B, D, N, L_total, chunk_L = 1, 256, 16, 2048, 1024
    x = _inputs(789, B, L_total, D, N, torch.float16)
    g = _dev(x, dev)
    with torch.no_grad():
        out_full, _ = kernel.forward_with_state(*_args(g), g["h_prev"])
        h = torch.zeros(B, D, N, device=dev, dtype=torch.float16)
        chunks = []
        for i in range(0, L_total, chunk_L):
            s = slice(i, min(i + chunk_L, L_total))
            out_c, h = kernel.forward_with_state(g["u"][:, s], g["delta"][:, s], g["A"], g["B"][:, s],
                                                 g["C"][:, s], g["D"], h_prev=h)
            chunks.append(out_c)
    out_stream = torch.cat(chunks, dim=1)
    assert (out_full.float() - out_stream.float()).abs().max().item() < 1e-3


def test_input_validation(dev, kernel):
    """test_selective_scan.py:239-262: h_prev with the wrong N or batch raises RuntimeError."""
    print("case reference input validation", flush=True)
    B, L, D, N = 1, 1024, 256, 16
    torch.manual_seed(0)
    u = torch.randn(B, L, D).half().to(dev)
    delta = torch.ones(B, L, D).half().to(dev)
    A = (-torch.rand(D, N) * 0.1).half().to(dev)
    B_ssm = torch.randn(B, L, N).half().to(dev)
    C_ssm = torch.randn(B, L, N).half().to(dev)
    D_ssm = torch.ones(D).half().to(dev)
    with pytest.raises(RuntimeError):
        kernel(u, delta, A, B_ssm, C_ssm, D_ssm, torch.randn(B, D, N + 1).half().to(dev))
    with pytest.raises(RuntimeError):
        kernel(u, delta, A, B_ssm, C_ssm, D_ssm, torch.randn(B + 1, D, N).half().to(dev))


def test_numerical_stability_extreme_values(dev, kernel):
    """test_selective_scan.py:264-285: delta = 10, fp16, the output stays finite (and matches)."""
    print("case reference extreme delta", flush=True)
    x = _inputs(999, 1, 512, 64, 16, torch.float16, delta_val=10.0)
    g = _dev(x, dev)
    with torch.no_grad():
        out = kernel(*_args(g), g["h_prev"])
    assert torch.isfinite(out).all()
    ref, _ = _oracle(x)
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, **TOL[torch.float16])


def test_gradient_flow(dev, kernel):
    """test_selective_scan.py:287-330: fp32, loss = out.sum() + h_last.sum(); every gradient,
    dh_prev included, exists and is finite."""
    print("case reference gradient flow", flush=True)
    x = _inputs(42, 1, 256, 64, 16, torch.float32)
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in x.items()}
    out, h_last = kernel.forward_with_state(*_args(leaves), leaves["h_prev"])
    (out.sum() + h_last.sum()).backward()
    for k, t in leaves.items():
        assert t.grad is not None, f"{k} grad is None"
        assert torch.isfinite(t.grad).all(), f"{k} grad contains NaN/Inf"


def test_gradient_numerical_accuracy(dev, kernel):
    """test_selective_scan.py:332-380: du and dA of loss = out.sum() + h_last.sum() against
    selective_scan_ref's autograd (fp32, bound 1e-3), and against the oracle's adjoint."""
    print("case reference gradient accuracy", flush=True)
    x = _inputs(123, 1, 128, 32, 16, torch.float32, h_prev=None)
    # this test draws u unscaled (test_selective_scan.py:341), unlike the others' 0.1 N(0,1)
    torch.manual_seed(123)
    x["u"] = torch.randn(1, 128, 32)
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in x.items()}
    out, h_last = kernel.forward_with_state(*_args(leaves))
    (out.sum() + h_last.sum()).backward()
    du, dA = leaves["u"].grad.clone(), leaves["A"].grad.clone()
    ref = {k: v.to(dev).requires_grad_(True) for k, v in x.items()}
    out_r, h_r = selective_scan_ref(*_args(ref))
    (out_r.sum() + h_r.sum()).backward()
    assert (du - ref["u"].grad).abs().max().item() < 1e-3
    assert (dA - ref["A"].grad).abs().max().item() < 1e-3
    o = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], torch.ones(1, 128, 32),
                    dh_last=torch.ones(1, 32, 16))
    np.testing.assert_allclose(du.cpu().double().numpy(), o["du"], **TOL[torch.float32])
    np.testing.assert_allclose(dA.cpu().double().numpy(), o["dA"], **TOL[torch.float32])


def test_parallel_scan_correctness(dev):
    """test_pscan.py:14-35: (B, D, L, N) = (2, 32, 128, 16), |A| < 1, bound 1e-4."""
    print("case reference pscan correctness", flush=True)
    torch.manual_seed(42)
    A = (torch.randn(2, 32, 128, 16).abs() * 0.1).to(dev)
    X = torch.randn(2, 32, 128, 16).to(dev)
    H = parallel_scan_fn(A, X)
    H_ref = parallel_scan_ref(A, X)
    assert (H - H_ref).abs().max().item() < 1e-4


def test_parallel_scan_gradient(dev):
    """test_pscan.py:37-62: gradients of H.sum() exist and are finite."""
    print("case reference pscan gradient", flush=True)
    torch.manual_seed(123)
    A = (torch.randn(1, 16, 64, 8) * 0.1).to(dev).requires_grad_(True)
    X = torch.randn(1, 16, 64, 8).to(dev).requires_grad_(True)
    parallel_scan_fn(A, X).sum().backward()
    assert A.grad is not None and X.grad is not None
    assert torch.isfinite(A.grad).all() and torch.isfinite(X.grad).all()
    dA, dX = orc.pscan_bwd(A, orc.pscan_fwd(A, X), np.ones((1, 16, 64, 8)))
    np.testing.assert_allclose(X.grad.cpu().double().numpy(), dX, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(A.grad.cpu().double().numpy(), dA, rtol=1e-5, atol=1e-5)


def test_parallel_scan_long_sequence(dev):
    """test_pscan.py:64-81: (1, 64, 1024, 16), shape kept and output finite."""
    print("case reference pscan long sequence", flush=True)
    torch.manual_seed(456)
    A = (torch.randn(1, 64, 1024, 16).abs() * 0.05).to(dev)
    X = torch.randn(1, 64, 1024, 16).to(dev)
    H = parallel_scan_fn(A, X)
    assert tuple(H.shape) == (1, 64, 1024, 16)
    assert torch.isfinite(H).all()
    np.testing.assert_allclose(H.cpu().double().numpy(), orc.pscan_fwd(A, X), rtol=1e-4, atol=1e-4)
