"""GPU parity of the reference API surfaces beyond SelectiveScanCuda.forward_with_state: the V1/V2
autograd Functions, forward(h_prev) returning out only, parallel_scan_fn's adjoint at the config-4b
length, the scan's bounded-wait error path, and the reference's long fp16 stream."""
import numpy as np
import pytest
import torch

from mamba_windows_cuda import SelectiveScanCuda, parallel_scan_fn, workloads
from mamba_windows_cuda.mamba_cuda import SelectiveScanFn, SelectiveScanFnV2
from mamba_windows_cuda.selective_scan_cuda_ext import FusedSelectiveScanFunction
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.float16: dict(rtol=1e-2, atol=1e-2)}
GRADS = (("u", "du"), ("delta", "ddelta"), ("A", "dA"), ("B", "dB"), ("C", "dC"), ("D", "dD"))


def _np(t):
    return t.detach().cpu().double().numpy()


@pytest.mark.parametrize("fn", [SelectiveScanFn, SelectiveScanFnV2], ids=["V1_recompute", "V2_save"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_v1_v2_functions(dev, fn, dtype):
    """SelectiveScanFn (reference V1, mamba_cuda.py:1099-1133) and SelectiveScanFnV2 (V2, 1136-1169):
    out and the six gradients against the float64 oracle, gradients in the input dtype."""
    print(f"case {fn.__name__} dtype={dtype}", flush=True)
    x = workloads.ssm_inputs(2, 300, 200, dtype=dtype, seed=31)
    leaves = {k: x[k].to(dev).requires_grad_(True) for k in ("u", "delta", "A", "B", "C", "D")}
    out = fn.apply(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"], leaves["D"])
    assert out.dtype == dtype and tuple(out.shape) == (2, 300, 200)
    out.backward(x["dout"].to(dev))
    torch.cuda.synchronize()
    ro, _ = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], None, clamp=True)
    np.testing.assert_allclose(_np(out), ro, err_msg="out", **TOL[dtype])
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], None, None, clamp=True)
    for k, name in GRADS:
        assert leaves[k].grad.dtype == dtype, name
        np.testing.assert_allclose(_np(leaves[k].grad), r[name], err_msg=name, **TOL[dtype])


@pytest.mark.parametrize("lvl", [0, 1])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_fused_selective_scan_function(dev, lvl, dtype):
    """FusedSelectiveScanFunction.apply(u, delta, A, B, C, D, h_prev, checkpoint_lvl) (the reference's
    class, selective_scan_cuda_ext.py:562-633) at both checkpoint levels: out, h_last, the six
    gradients and dh_prev against the float64 oracle, with an upstream gradient on h_last too."""
    print(f"case FusedSelectiveScanFunction lvl={lvl} dtype={dtype}", flush=True)
    x = workloads.ssm_inputs(2, 260, 150, dtype=dtype, h_prev=True, seed=33)
    dhl = (0.5 * torch.randn(2, 150, 16, generator=torch.Generator().manual_seed(34))).to(dtype)
    names = ("u", "delta", "A", "B", "C", "D", "h_prev")
    leaves = {k: x[k].to(dev).requires_grad_(True) for k in names}
    out, h_last = FusedSelectiveScanFunction.apply(*(leaves[k] for k in names), lvl)
    assert out.dtype == dtype and tuple(h_last.shape) == (2, 150, 16)
    torch.autograd.backward([out, h_last], [x["dout"].to(dev), dhl.to(dev)])
    torch.cuda.synchronize()
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True)
    np.testing.assert_allclose(_np(out), ro, err_msg="out", **TOL[dtype])
    np.testing.assert_allclose(_np(h_last), rh, err_msg="h_last", **TOL[dtype])
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], dhl, clamp=True)
    for k, name in GRADS + (("h_prev", "dh_prev"),):
        assert leaves[k].grad.dtype == dtype, name
        np.testing.assert_allclose(_np(leaves[k].grad), r[name], err_msg=name, **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_forward_with_h_prev_returns_out_only(dev, dtype):
    """SelectiveScanCuda.forward(..., h_prev) returns out alone (reference mamba_cuda.py:1190-1194), and
    its backward reaches h_prev: dh_prev and the six gradients against the oracle."""
    print(f"case forward(h_prev) dtype={dtype}", flush=True)
    x = workloads.ssm_inputs(3, 150, 96, dtype=dtype, h_prev=True, seed=32)
    names = ("u", "delta", "A", "B", "C", "D", "h_prev")
    leaves = {k: x[k].to(dev).requires_grad_(True) for k in names}
    out = SelectiveScanCuda()(*(leaves[k] for k in names))
    assert isinstance(out, torch.Tensor) and tuple(out.shape) == (3, 150, 96)
    out.backward(x["dout"].to(dev))
    torch.cuda.synchronize()
    ro, _ = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True)
    np.testing.assert_allclose(_np(out), ro, err_msg="out", **TOL[dtype])
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], None, clamp=True)
    for k, name in GRADS + (("h_prev", "dh_prev"),):
        np.testing.assert_allclose(_np(leaves[k].grad), r[name], err_msg=name, **TOL[dtype])


def test_pscan_adjoint_config4b_length(dev):
    """parallel_scan_fn forward and adjoint over one full config-4b sequence, (1, 65536, 1024) fp32:
    512 tiles chained by the look-back in each direction, against the float64 scan and its adjoint."""
    a, b = workloads.pscan_inputs((1, 65536, 1024), seed=3)
    dH = torch.randn(1, 65536, 1024, generator=torch.Generator().manual_seed(4))
    ad = a.to(dev).requires_grad_(True)
    bd = b.to(dev).requires_grad_(True)
    H = parallel_scan_fn(ad, bd)
    H.backward(dH.to(dev))
    torch.cuda.synchronize()
    ref = orc.pscan_fwd(a, b)
    np.testing.assert_allclose(_np(H), ref, rtol=1e-3, atol=1e-4)
    rdA, rdX = orc.pscan_bwd(a, torch.from_numpy(ref), dH)
    np.testing.assert_allclose(_np(bd.grad), rdX, rtol=1e-3, atol=1e-4)
    np.testing.assert_allclose(_np(ad.grad), rdA, rtol=1e-3, atol=1e-4)


def test_pscan_wait_give_up_is_reported(dev, monkeypatch):
    """A look-back wait that runs out of polls is an error, not a silently wrong H: with a limit of 0
    every wait gives up at once (each kernel still runs to its end) and the tiles that waited hold
    NaN. The scan calls read their status words without waiting: pscan_check() reports the failure
    at once, and the first scan call after it finished reports it too. The default limit gives OK."""
    from mamba_windows_cuda import _lib, ops
    from mamba_windows_cuda.pscan import pscan_check

    a, b = workloads.pscan_inputs((2, 1000, 64), seed=5)
    ad, bd = a.to(dev), b.to(dev)
    H = parallel_scan_fn(ad, bd)  # default limit: completes
    pscan_check()
    np.testing.assert_allclose(_np(H), orc.pscan_fwd(a, b), rtol=1e-3, atol=1e-4)

    monkeypatch.setenv("MWC_PSCAN_SPIN_LIMIT", "0")
    Hbad = parallel_scan_fn(ad, bd)  # enqueued; its status word is read without waiting
    with pytest.raises(RuntimeError, match="MWC_ERR_INCOMPLETE"):
        pscan_check()
    assert torch.isnan(Hbad[:, 128:]).all()
    parallel_scan_fn(ad, bd)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="MWC_ERR_INCOMPLETE"):
        parallel_scan_fn(ad, bd)  # reports the finished failure of the call before
    # the raw C ABI: the waiting and the non-waiting status reads; the first tile (no predecessor) is
    # exact while later ones are NaN
    L_ = _lib.lib()
    nbytes = L_.mwc_pscan_workspace_size(2, 1000, 64)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    Hc = torch.empty_like(bd)
    st = L_.mwc_pscan_fwd(_lib.MWC_DTYPE_F32, ad.data_ptr(), bd.data_ptr(), Hc.data_ptr(), 2, 1000, 64,
                          ws.data_ptr(), nbytes, ops._stream(ad.device))
    assert st == 0
    word = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    assert L_.mwc_pscan_status_async(ws.data_ptr(), nbytes, 2, 1000, 64, word.data_ptr(),
                                     ops._stream(ad.device)) == 0
    assert L_.mwc_pscan_status(ws.data_ptr(), nbytes, 2, 1000, 64, ops._stream(ad.device)) == 5
    assert int(word[0]) != 0
    Hc = Hc.cpu()
    assert torch.isnan(Hc[:, 128:]).all()
    torch.testing.assert_close(Hc[:, :128], H[:, :128].cpu(), rtol=0, atol=0)
    monkeypatch.delenv("MWC_PSCAN_SPIN_LIMIT")
    Hd = parallel_scan_fn(ad, bd)  # the next call with the default limit clears the word and completes
    pscan_check()
    # (not bitwise: a tile's prefix sums its predecessors' aggregates or takes an inclusive prefix,
    # whichever is published when it looks, so the rounding order varies from run to run)
    torch.testing.assert_close(Hd, H, rtol=1e-5, atol=1e-5)


def test_long_fp16_stream(dev):
    """The reference's long-stream case (tests/test_selective_scan.py:218-237): 1280^2 fp16 steps fed in
    16384-step chunks through forward_with_state at D=2048, so h_last is rounded to fp16 at ~100
    chunk boundaries. Outputs and state stay finite, the streamed h equals one full-length pass, and
    the float64 oracle over the whole sequence agrees on a 16-channel slice (u ~ 0.1 N(0,1),
    delta = 0.01, A = -0.1 U(0,1), B, C ~ 0.1 N(0,1), D = 0.1, as the reference test draws them)."""
    Bsz, D, N = 1, 2048, 16
    L_total, chunk = 1280 * 1280, 16384
    g = torch.Generator(device=dev).manual_seed(11)
    u = (0.1 * torch.randn(Bsz, L_total, D, generator=g, device=dev)).half()
    delta = torch.full((Bsz, L_total, D), 0.01, device=dev).half()
    A = (-0.1 * torch.rand(D, N, generator=g, device=dev)).half()
    Bs = (0.1 * torch.randn(Bsz, L_total, N, generator=g, device=dev)).half()
    Cs = (0.1 * torch.randn(Bsz, L_total, N, generator=g, device=dev)).half()
    Dv = torch.full((D,), 0.1, device=dev).half()
    m = SelectiveScanCuda()
    h = torch.zeros(Bsz, D, N, device=dev).half()
    nchunks = (L_total + chunk - 1) // chunk
    print(f"case long fp16 stream: {nchunks} chunks", flush=True)
    with torch.no_grad():
        for s in range(nchunks):
            sl = slice(s * chunk, min(L_total, (s + 1) * chunk))
            out, h = m.forward_with_state(u[:, sl], delta[:, sl], A, Bs[:, sl], Cs[:, sl], Dv, h)
            if s == nchunks - 1:
                last_out = out
        _, h_full = m.forward_with_state(u, delta, A, Bs, Cs, Dv, None)
    torch.cuda.synchronize()
    assert torch.isfinite(last_out).all() and torch.isfinite(h).all()
    torch.testing.assert_close(h, h_full, **TOL[torch.float16])
    k = 16
    ro, rh = orc.ssm_fwd(u[:, :, :k].cpu(), delta[:, :, :k].cpu(), A[:k].cpu(), Bs.cpu(), Cs.cpu(), Dv[:k].cpu(),
                         None, clamp=True)
    np.testing.assert_allclose(_np(h[:, :k]), rh, **TOL[torch.float16])
    np.testing.assert_allclose(_np(h_full[:, :k]), rh, **TOL[torch.float16])
    np.testing.assert_allclose(_np(last_out[:, :, :k]), ro[:, -last_out.shape[1]:], **TOL[torch.float16])


@pytest.mark.parametrize("shape", [(1, 16384, 768), (1, 16384, 1024), (1, 32768, 2048)])
def test_long_fp16_single_pass(dev, shape):
    """The reference's long single passes (tests/test_selective_scan.py:195-213): fp16 forward at
    L = 16384 and 32768 (u, B, C ~ 0.1 N(0,1), delta = 0.01, A = -0.1 U(0,1), D = 0.1). The output is
    finite, and on a 16-channel slice it matches the float64 oracle over the whole sequence."""
    Bsz, L, D = shape
    N = 16
    print(f"case long fp16 single pass {shape}", flush=True)
    g = torch.Generator(device=dev).manual_seed(123)
    u = (0.1 * torch.randn(Bsz, L, D, generator=g, device=dev)).half()
    delta = torch.full((Bsz, L, D), 0.01, device=dev).half()
    A = (-0.1 * torch.rand(D, N, generator=g, device=dev)).half()
    Bs = (0.1 * torch.randn(Bsz, L, N, generator=g, device=dev)).half()
    Cs = (0.1 * torch.randn(Bsz, L, N, generator=g, device=dev)).half()
    Dv = torch.full((D,), 0.1, device=dev).half()
    with torch.no_grad():
        out = SelectiveScanCuda()(u, delta, A, Bs, Cs, Dv)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and torch.isfinite(out).all()
    k = 16
    ro, _ = orc.ssm_fwd(u[:, :, :k].cpu(), delta[:, :, :k].cpu(), A[:k].cpu(), Bs.cpu(), Cs.cpu(), Dv[:k].cpu(),
                        None, clamp=True)
    np.testing.assert_allclose(_np(out[:, :, :k]), ro, **TOL[torch.float16])


def test_beyond_2_31_elements(dev):
    """B*L*D = 2^32 fp16 elements (B=2, L=2^20, D=2048; batch row 1 starts 2^31 elements in): the fused
    forward and backward address every tensor with 64-bit offsets. Checked by a property of the scan:
    the last 4096 steps of row 1 equal a separate fp32 call on those steps started from the forward's
    checkpoint state, and so do their du, ddelta, dB and dC (the adjoint at a step depends only on later
    steps). The inputs take ~26 GB, the whole step ~90 GB of the 288 GB HBM."""
    from mamba_windows_cuda import ops

    Bsz, L, D, N, T = 2, 1 << 20, 2048, 16, 4096
    print(f"case beyond 2^31 elements B={Bsz} L={L} D={D}", flush=True)
    g = torch.Generator(device=dev).manual_seed(31)
    u = torch.randn(Bsz, L, D, generator=g, device=dev, dtype=torch.float16)
    delta = torch.rand(Bsz, L, D, generator=g, device=dev, dtype=torch.float16).mul_(0.099).add_(0.001)
    A = -(0.01 + 0.99 * torch.rand(D, N, generator=g, device=dev)).half()
    Bs = torch.randn(Bsz, L, N, generator=g, device=dev, dtype=torch.float16)
    Cs = torch.randn(Bsz, L, N, generator=g, device=dev, dtype=torch.float16)
    Dv = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).half()
    out, _, ckpt = ops.ssm_forward(u, delta, A, Bs, Cs, Dv, want_h_last=False, want_ckpt=True)
    t0 = L - T
    h0 = ckpt[1:2, t0 // 16].clone()  # fp32 state before step t0 of row 1
    tail = [t[1:2, t0:].float() for t in (u, delta)] + [A.float()] + [t[1:2, t0:].float() for t in (Bs, Cs)] + \
        [Dv.float()]
    ref_out, _, ref_ckpt = ops.ssm_forward(*tail, h0, want_h_last=False, want_ckpt=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out[1, t0:]).all()
    torch.testing.assert_close(out[1:2, t0:].float(), ref_out, **TOL[torch.float16])
    dout = torch.randn(Bsz, L, D, generator=g, device=dev, dtype=torch.float16)
    du, ddelta, _, dB, dC, _, _ = ops.ssm_backward(u, delta, A, Bs, Cs, Dv, dout, ckpt)
    del ckpt
    rdu, rdd, _, rdB, rdC, _, _ = ops.ssm_backward(*tail, dout[1:2, t0:].float(), ref_ckpt, None, False)
    torch.cuda.synchronize()
    for name, got, ref in (("du", du, rdu), ("ddelta", ddelta, rdd), ("dB", dB, rdB), ("dC", dC, rdC)):
        assert torch.isfinite(got[1, t0:]).all(), name
        torch.testing.assert_close(got[1:2, t0:].float(), ref, msg=name, **TOL[torch.float16])
    del u, delta, dout, out, du, ddelta
    torch.cuda.empty_cache()  # hand the ~90 GB back before the next test
