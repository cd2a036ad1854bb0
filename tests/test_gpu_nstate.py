"""GPU parity of the scan, its backward and the decode step at state counts N = 8, 32, 64.

The reference builds N = 16 only (mamba_cuda.py:215); the kernels here are templated on N, so
every other count gets the same checks as N = 16 against the float64 oracle, which is written
for any N: out, h_last and every gradient (incl. dh_prev), over the lane-group widths the
launcher picks for small and large B*D, with L split into segments, with the fused transforms,
in fp32/fp16/bf16, and one decode step. Tolerances as in test_gpu_ssm.py.
"""
import numpy as np
import pytest
import torch

from mamba_windows_cuda import SelectiveScanCuda, workloads
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.float16: dict(rtol=1e-2, atol=1e-2),
       torch.bfloat16: dict(rtol=2e-2, atol=2e-2)}
GRADS = (("u", "du"), ("delta", "ddelta"), ("A", "dA"), ("B", "dB"), ("C", "dC"), ("D", "dD"),
         ("h_prev", "dh_prev"))
NS = [8, 32, 64]


def _close(name, got, ref, dtype):
    np.testing.assert_allclose(got.detach().cpu().double().numpy(), ref, err_msg=name, **TOL[dtype])


def _inputs(B, L, D, n, dtype, seed, xf=False):
    x = workloads.ssm_inputs(B, L, D, dtype=torch.float32, h_prev=True, seed=seed, nstate=n)
    g = torch.Generator().manual_seed(seed + 1)
    x["dh_last"] = 0.5 * torch.randn(B, D, n, generator=g)
    if xf:
        x["delta"] = -4.0 + 2.0 * torch.randn(B, L, D, generator=g)
        x["delta_bias"] = 0.5 * torch.randn(D, generator=g)
        x["z"] = torch.randn(B, L, D, generator=g)
    return {k: v.to(dtype) for k, v in x.items()}


def _check(dev, x, dtype, *, xf=False, lvl=0):
    names = ["u", "delta", "A", "B", "C", "D", "h_prev"] + (["delta_bias", "z"] if xf else [])
    leaves = {k: x[k].to(dev).requires_grad_(True) for k in names}
    out, h_last = SelectiveScanCuda(checkpoint_lvl=lvl).forward_with_state(
        leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"], leaves["D"], leaves["h_prev"],
        z=leaves.get("z"), delta_bias=leaves.get("delta_bias"), delta_softplus=xf)
    loss = (out.float() * x["dout"].to(dev).float()).sum() + (h_last.float() * x["dh_last"].to(dev).float()).sum()
    loss.backward()
    torch.cuda.synchronize()
    kw = dict(delta_bias=x["delta_bias"], delta_softplus=True, z=x["z"]) if xf else {}
    ro, rh, _ = orc.ssm_fwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True, **kw)
    _close("out", out, ro, dtype)
    _close("h_last", h_last, rh, dtype)
    r = orc.ssm_bwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], x["dh_last"],
                       clamp=True, **kw)
    for k, name in GRADS:
        _close(name, leaves[k].grad, r[name], dtype)
    if xf:
        _close("ddelta_bias", leaves["delta_bias"].grad, r["ddelta_bias"], dtype)
        _close("dz", leaves["z"].grad, r["dz"], dtype)


@pytest.mark.parametrize("n", NS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("shape", [(1, 77, 70), (2, 45, 1100), (3, 40, 2100)])
def test_scan_parity(dev, n, dtype, shape):
    B, L, D = shape
    print(f"case nstate={n} shape={shape} dtype={dtype}", flush=True)
    _check(dev, _inputs(B, L, D, n, dtype, seed=n + B + L + D), dtype)


# (N, states per lane, segments of L, carry segments per segment): every built lane group
PLANS = [(8, 1, 3, 2), (8, 2, 2, 1), (32, 2, 4, 2), (32, 4, 3, 1), (64, 4, 5, 2)]


@pytest.mark.parametrize("plan", PLANS)
def test_segmented_plans(dev, monkeypatch, plan):
    n, spl, nseg, cfold = plan
    monkeypatch.setenv("MWC_SPL", str(spl))
    monkeypatch.setenv("MWC_NSEG", str(nseg))
    monkeypatch.setenv("MWC_CFOLD", str(cfold))
    print(f"case nstate segmented plan={plan}", flush=True)
    _check(dev, _inputs(2, 333, 200, n, torch.float32, seed=nseg * 10 + n), torch.float32)


@pytest.mark.parametrize("n", NS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_transforms(dev, monkeypatch, n, dtype):
    monkeypatch.setenv("MWC_NSEG", "3")
    print(f"case nstate={n} transforms dtype={dtype}", flush=True)
    _check(dev, _inputs(2, 200, 96, n, dtype, seed=n + 5, xf=True), dtype, xf=True)


@pytest.mark.parametrize("n", NS)
def test_checkpoint_levels_agree(dev, n):
    """Level 1 (rebuild the checkpoints in the backward) matches level 0 bitwise."""
    x = _inputs(2, 150, 80, n, torch.float32, seed=n + 9, xf=True)
    outs = []
    for lvl in (0, 1):
        leaves = {k: x[k].to(dev).requires_grad_(True) for k in ("u", "delta", "A", "B", "C", "D", "h_prev", "z")}
        out, hl = SelectiveScanCuda(checkpoint_lvl=lvl).forward_with_state(
            leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"], leaves["D"], leaves["h_prev"],
            z=leaves["z"], delta_softplus=True)
        (out.float() * x["dout"].to(dev)).sum().backward()
        outs.append([out, hl] + [leaves[k].grad for k in leaves])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("n", NS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_step(dev, n, dtype):
    Bsz, D = 3, 500
    print(f"case nstate={n} step dtype={dtype}", flush=True)
    x = _inputs(Bsz, 1, D, n, dtype, seed=n + 2, xf=True)
    xd = {k: v.to(dev) for k, v in x.items()}
    with torch.no_grad():
        y, h = SelectiveScanCuda().step(xd["u"][:, 0], xd["delta"][:, 0], xd["A"], xd["B"][:, 0], xd["C"][:, 0],
                                        xd["D"], xd["h_prev"], z=xd["z"][:, 0], delta_bias=xd["delta_bias"],
                                        delta_softplus=True)
    ro, rh, _ = orc.ssm_fwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True,
                               delta_bias=x["delta_bias"], delta_softplus=True, z=x["z"])
    _close("out", y, ro[:, 0], dtype)
    _close("h_new", h, rh, dtype)
