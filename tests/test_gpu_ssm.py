"""GPU parity of the fused selective-scan kernels against the float64 oracle.

Inputs are generated on the CPU (seeded), cast to the test dtype, and the
oracle runs in float64 on exactly those dtype-rounded values. Tolerances
(|x - y| <= atol + rtol*|y|): fp32 rtol 1e-3 / atol 1e-4, fp16 rtol 1e-2 /
atol 1e-2, applied to out, h_last and every gradient.
"""
import numpy as np
import pytest
import torch

from mamba_windows_cuda import FusedSelectiveScan, SelectiveScanCuda, workloads
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

# bf16 (8-bit mantissa; not in the reference) rounds outputs ~8x coarser than fp16: twice fp16's bound
TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.float16: dict(rtol=1e-2, atol=1e-2),
       torch.bfloat16: dict(rtol=2e-2, atol=2e-2)}
GRADS = (("u", "du"), ("delta", "ddelta"), ("A", "dA"), ("B", "dB"), ("C", "dC"), ("D", "dD"))


def _np(t):
    return t.detach().cpu().double().numpy()


def _close(name, got, ref, dtype):
    np.testing.assert_allclose(_np(got), ref, err_msg=name, **TOL[dtype])


def _run(x, dev, *, with_h, dh_last=None, lvl=0, grads=True):
    """forward_with_state + backward through the drop-in API; returns out, h_last, grads dict."""
    leaves = {k: v.to(dev).requires_grad_(grads and k not in ("dout",)) for k, v in x.items()}
    m = SelectiveScanCuda(checkpoint_lvl=lvl)
    out, h_last = m.forward_with_state(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"],
                                       leaves["D"], leaves["h_prev"] if with_h else None)
    g = {}
    if grads:
        loss = (out.float() * leaves["dout"].float()).sum()
        if dh_last is not None:
            loss = loss + (h_last.float() * dh_last.to(dev).float()).sum()
        loss.backward()
        g = {k: leaves[k].grad for k in leaves if leaves[k].grad is not None}
    torch.cuda.synchronize()
    return out, h_last, g


# (B, L, D): lane-group widths 1/2/4 states per lane are chosen by B*D; ragged D and L on purpose.
SHAPES = [(1, 77, 70), (2, 45, 1100), (4, 33, 2100), (3, 1, 20), (1, 16, 16), (2, 130, 64)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("with_h", [False, True])
def test_forward_backward_parity(dev, shape, dtype, with_h):
    B, L, D = shape
    print(f"case fwd+bwd shape={shape} dtype={dtype} h_prev={with_h}", flush=True)
    x = workloads.ssm_inputs(B, L, D, dtype=dtype, h_prev=True, seed=B * 1000 + L + D)
    dhl = (0.5 * torch.randn(B, D, 16, generator=torch.Generator().manual_seed(3))).to(dtype) if with_h else None
    out, h_last, g = _run(x, dev, with_h=with_h, dh_last=dhl)
    hp = x["h_prev"] if with_h else None
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], hp, clamp=True)
    _close("out", out, ro, dtype)
    _close("h_last", h_last, rh, dtype)
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], hp, dhl, clamp=True)
    for k, name in GRADS:
        _close(name, g[k], r[name], dtype)
    if with_h:
        _close("dh_prev", g["h_prev"], r["dh_prev"], dtype)


# Forced launch plans: states per lane x segments of L x carry segments per segment.
PLANS = [(1, 1, 1), (1, 3, 1), (1, 4, 2), (2, 2, 1), (2, 5, 4), (4, 3, 2), (2, 64, 1)]


@pytest.mark.parametrize("plan", PLANS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_segmented_plans(dev, monkeypatch, plan, dtype):
    """L split into segments (carry pass + main pass): same results as the oracle, incl. h_prev/dh_last."""
    spl, nseg, cfold = plan
    monkeypatch.setenv("MWC_SPL", str(spl))
    monkeypatch.setenv("MWC_NSEG", str(nseg))
    monkeypatch.setenv("MWC_CFOLD", str(cfold))
    B, L, D = 2, 333, 200
    print(f"case segmented plan={plan} dtype={dtype}", flush=True)
    x = workloads.ssm_inputs(B, L, D, dtype=dtype, h_prev=True, seed=17 + nseg)
    dhl = (0.5 * torch.randn(B, D, 16, generator=torch.Generator().manual_seed(4))).to(dtype)
    out, h_last, g = _run(x, dev, with_h=True, dh_last=dhl)
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True)
    _close("out", out, ro, dtype)
    _close("h_last", h_last, rh, dtype)
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], dhl, clamp=True)
    for k, name in GRADS:
        _close(name, g[k], r[name], dtype)
    _close("dh_prev", g["h_prev"], r["dh_prev"], dtype)


def test_segmented_clamp_path(dev, monkeypatch):
    """Segments whose carries take the clamped exponent path (|delta*A| > 88 in some chunks)."""
    monkeypatch.setenv("MWC_NSEG", "4")
    monkeypatch.setenv("MWC_CFOLD", "2")
    B, L, D = 1, 256, 64
    x = workloads.ssm_inputs(B, L, D, dtype=torch.float32, h_prev=True, seed=23)
    x["delta"][:, 40:60] *= 2000.0  # delta up to 200 with |A| up to 1: exponents beyond -88
    x["delta"][:, 150:151] *= 5000.0
    dhl = torch.randn(B, D, 16, generator=torch.Generator().manual_seed(5))
    out, h_last, g = _run(x, dev, with_h=True, dh_last=dhl)
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True)
    _close("out", out, ro, torch.float32)
    _close("h_last", h_last, rh, torch.float32)
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], dhl, clamp=True)
    for k, name in GRADS:
        _close(name, g[k], r[name], torch.float32)
    _close("dh_prev", g["h_prev"], r["dh_prev"], torch.float32)


def _run_xf(x, dev, *, bias, softplus, gate, lvl=0, dh_last=None):
    """forward_with_state with the fused transforms + backward; returns out, h_last, grads."""
    names = ["u", "delta", "A", "B", "C", "D", "h_prev"] + (["delta_bias"] if bias else []) + (["z"] if gate else [])
    leaves = {k: x[k].to(dev).requires_grad_(True) for k in names}
    m = SelectiveScanCuda(checkpoint_lvl=lvl)
    out, h_last = m.forward_with_state(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"],
                                       leaves["D"], leaves["h_prev"], z=leaves.get("z"),
                                       delta_bias=leaves.get("delta_bias"), delta_softplus=softplus)
    loss = (out.float() * x["dout"].to(dev).float()).sum()
    if dh_last is not None:
        loss = loss + (h_last.float() * dh_last.to(dev).float()).sum()
    loss.backward()
    torch.cuda.synchronize()
    return out, h_last, {k: v.grad for k, v in leaves.items()}


XF_CASES = [(True, True, True), (True, True, False), (False, False, True), (False, True, False), (True, False, False)]


@pytest.mark.parametrize("xf", XF_CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("shape,nseg", [((2, 333, 200), "3"), ((1, 77, 70), None), ((3, 40, 2100), None)])
def test_fused_transforms(dev, monkeypatch, xf, dtype, shape, nseg):
    """delta' = softplus(delta + delta_bias) and out * silu(z) fused into the kernels: out, h_last and
    every gradient (incl. delta_bias, z, h_prev) against the float64 oracle composed with the
    transforms."""
    bias, softplus, gate = xf
    if nseg:
        monkeypatch.setenv("MWC_NSEG", nseg)
    B, L, D = shape
    print(f"case transforms xf={xf} dtype={dtype} shape={shape} nseg={nseg}", flush=True)
    x = workloads.ssm_inputs(B, L, D, dtype=torch.float32, h_prev=True, seed=B + L + D)
    g = torch.Generator().manual_seed(7)
    if softplus:  # raw delta around softplus^-1 of the usual range
        x["delta"] = -4.0 + 2.0 * torch.randn(B, L, D, generator=g)
    x["delta_bias"] = 0.5 * torch.randn(D, generator=g)
    if not softplus:  # without softplus delta + bias must stay a step size (> 0), or the states grow
        x["delta_bias"] = 0.1 * x["delta_bias"].abs()
    x["z"] = torch.randn(B, L, D, generator=g)
    x = {k: v.to(dtype) for k, v in x.items()}
    dhl = (0.5 * torch.randn(B, D, 16, generator=g)).to(dtype)
    out, h_last, gr = _run_xf(x, dev, bias=bias, softplus=softplus, gate=gate, dh_last=dhl)
    kw = dict(delta_bias=x["delta_bias"] if bias else None, delta_softplus=softplus, z=x["z"] if gate else None,
              clamp=True)
    ro, rh, _ = orc.ssm_fwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], **kw)
    _close("out", out, ro, dtype)
    _close("h_last", h_last, rh, dtype)
    r = orc.ssm_bwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], dhl, **kw)
    for k, name in GRADS + (("h_prev", "dh_prev"),):
        _close(name, gr[k], r[name], dtype)
    if bias:
        _close("ddelta_bias", gr["delta_bias"], r["ddelta_bias"], dtype)
    if gate:
        _close("dz", gr["z"], r["dz"], dtype)


def test_fused_transforms_wide_delta(dev, monkeypatch):
    """softplus over its whole range: raw delta + bias from about -40 to +35, so every branch of the
    kernels' softplus (x itself above 20, the log2 form, the series for e^x < 2^-6) and the
    derivative past the threshold are taken; fp32, L split into segments, ragged last chunk."""
    monkeypatch.setenv("MWC_NSEG", "3")
    B, L, D = 2, 203, 96
    x = workloads.ssm_inputs(B, L, D, dtype=torch.float32, h_prev=True, seed=31)
    g = torch.Generator().manual_seed(11)
    x["delta"] = -4.0 + 9.0 * torch.randn(B, L, D, generator=g)
    x["delta_bias"] = 0.5 * torch.randn(D, generator=g)
    x["z"] = torch.randn(B, L, D, generator=g)
    pre = x["delta"] + x["delta_bias"]
    assert (pre > 20).any() and (pre < -10).any()
    dhl = 0.5 * torch.randn(B, D, 16, generator=g)
    out, h_last, gr = _run_xf(x, dev, bias=True, softplus=True, gate=True, dh_last=dhl)
    kw = dict(delta_bias=x["delta_bias"], delta_softplus=True, z=x["z"], clamp=True)
    ro, rh, _ = orc.ssm_fwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], **kw)
    _close("out", out, ro, torch.float32)
    _close("h_last", h_last, rh, torch.float32)
    r = orc.ssm_bwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], dhl, **kw)
    for k, name in GRADS + (("h_prev", "dh_prev"),):
        _close(name, gr[k], r[name], torch.float32)
    _close("ddelta_bias", gr["delta_bias"], r["ddelta_bias"], torch.float32)
    _close("dz", gr["z"], r["dz"], torch.float32)


def test_fused_transforms_levels_agree(dev):
    """Checkpoint levels 0 and 1 give bitwise-equal results with all three transforms."""
    x = workloads.ssm_inputs(2, 300, 96, dtype=torch.float32, h_prev=True, seed=9)
    g = torch.Generator().manual_seed(8)
    x["delta"] = -3.0 + torch.randn(2, 300, 96, generator=g)
    x["delta_bias"] = torch.randn(96, generator=g)
    x["z"] = torch.randn(2, 300, 96, generator=g)
    o0, h0, g0 = _run_xf(x, dev, bias=True, softplus=True, gate=True, lvl=0)
    o1, h1, g1 = _run_xf(x, dev, bias=True, softplus=True, gate=True, lvl=1)
    assert torch.equal(o0, o1) and torch.equal(h0, h1)
    for k in g0:
        assert torch.equal(g0[k], g1[k]), k


@pytest.mark.parametrize("shape,nseg", [((1, 77, 70), None), ((2, 333, 200), "3"), ((3, 40, 2100), None)])
@pytest.mark.parametrize("xf", [False, True])
def test_bfloat16(dev, monkeypatch, shape, nseg, xf):
    """bf16 storage (fp32 math): out, h_last and every gradient against the float64 oracle on the
    bf16-rounded inputs, with and without the fused transforms, split and unsplit."""
    if nseg:
        monkeypatch.setenv("MWC_NSEG", nseg)
    B, L, D = shape
    print(f"case bf16 shape={shape} nseg={nseg} xf={xf}", flush=True)
    x = workloads.ssm_inputs(B, L, D, dtype=torch.float32, h_prev=True, seed=B * 7 + L + D)
    g = torch.Generator().manual_seed(2)
    x["delta_bias"] = 0.5 * torch.randn(D, generator=g)
    x["z"] = torch.randn(B, L, D, generator=g)
    if xf:
        x["delta"] = -4.0 + 2.0 * torch.randn(B, L, D, generator=g)
    x = {k: v.to(torch.bfloat16) for k, v in x.items()}
    dhl = (0.5 * torch.randn(B, D, 16, generator=g)).to(torch.bfloat16)
    out, h_last, gr = _run_xf(x, dev, bias=xf, softplus=xf, gate=xf, dh_last=dhl)
    kw = dict(delta_bias=x["delta_bias"] if xf else None, delta_softplus=xf, z=x["z"] if xf else None, clamp=True)
    ro, rh, _ = orc.ssm_fwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], **kw)
    _close("out", out, ro, torch.bfloat16)
    _close("h_last", h_last, rh, torch.bfloat16)
    r = orc.ssm_bwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], dhl, **kw)
    for k, name in GRADS + (("h_prev", "dh_prev"),):
        _close(name, gr[k], r[name], torch.bfloat16)
    if xf:
        _close("ddelta_bias", gr["delta_bias"], r["ddelta_bias"], torch.bfloat16)
        _close("dz", gr["z"], r["dz"], torch.bfloat16)


def test_checkpoint_levels_agree_bitwise(dev):
    x = workloads.ssm_inputs(2, 300, 96, dtype=torch.float32, h_prev=True, seed=5)
    _, _, g0 = _run(x, dev, with_h=True, lvl=0)
    _, _, g1 = _run(x, dev, with_h=True, lvl=1)
    for k in g0:
        assert torch.equal(g0[k], g1[k]), k
    f0 = FusedSelectiveScan(0).to(dev)
    f1 = FusedSelectiveScan(1).to(dev)
    xd = {k: v.to(dev) for k, v in x.items()}
    o0 = f0(xd["u"], xd["delta"], xd["A"], xd["B"], xd["C"], xd["D"])
    o1, _ = f1.forward_with_state(xd["u"], xd["delta"], xd["A"], xd["B"], xd["C"], xd["D"])
    assert torch.equal(o0, o1)


def test_repeatable(dev):
    x = workloads.ssm_inputs(2, 200, 2100, dtype=torch.float16, seed=6)
    o1, _, g1 = _run(x, dev, with_h=False)
    o2, _, g2 = _run(x, dev, with_h=False)
    assert torch.equal(o1, o2)
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k


def test_config0_forward(dev):
    x = workloads.config_inputs("cfg0")
    out, h_last, _ = _run(x, dev, with_h=False, grads=False)
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], None, clamp=True)
    _close("out", out, ro, torch.float32)
    _close("h_last", h_last, rh, torch.float32)


def test_config1_stateful_forward(dev):
    x = workloads.config_inputs("cfg1")
    out, h_last, _ = _run(x, dev, with_h=True, grads=False)
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True)
    _close("out", out, ro, torch.float16)
    _close("h_last", h_last, rh, torch.float16)


def test_config2_training_step(dev):
    """Mamba-130M layer shape, fp16: out and all six gradients vs the float64 oracle."""
    x = workloads.config_inputs("cfg2")
    out, _, g = _run(x, dev, with_h=False)
    ro, _ = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], None, clamp=True)
    _close("out", out, ro, torch.float16)
    del ro
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], None, None, clamp=True)
    for k, name in GRADS:
        _close(name, g[k], r[name], torch.float16)


def test_streaming_equals_full_pass(dev):
    """Chunks carried through h_prev -> h_last reproduce one full pass (reference
    tests/test_selective_scan.py:148-193, which bounds the max difference by 1e-3), here in fp32
    with config-2 distributions. The full pass may split L into segments whose carries are
    combined in a different order than the stream's, so the bound is rounding-level, not bitwise."""
    x = workloads.ssm_inputs(2, 1024, 256, dtype=torch.float32, seed=7, dout=False)
    xd = {k: v.to(dev) for k, v in x.items()}
    m = SelectiveScanCuda()
    with torch.no_grad():
        full, h_full = m.forward_with_state(xd["u"], xd["delta"], xd["A"], xd["B"], xd["C"], xd["D"])
        h = None
        outs = []
        for s in range(0, 1024, 256):
            sl = slice(s, s + 256)
            o, h = m.forward_with_state(xd["u"][:, sl], xd["delta"][:, sl], xd["A"], xd["B"][:, sl],
                                        xd["C"][:, sl], xd["D"], h)
            outs.append(o)
    torch.testing.assert_close(torch.cat(outs, 1), full, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(h, h_full, rtol=1e-4, atol=1e-5)


def test_stateful_gradient_chain(dev):
    """Gradients flow through h_last -> h_prev across two chunks exactly like one pass."""
    x = workloads.ssm_inputs(1, 96, 40, dtype=torch.float32, seed=8)
    xd = {k: v.to(dev).requires_grad_(k != "dout") for k, v in x.items()}
    m = SelectiveScanCuda()
    o1, h1 = m.forward_with_state(xd["u"][:, :50], xd["delta"][:, :50], xd["A"], xd["B"][:, :50],
                                  xd["C"][:, :50], xd["D"])
    o2, _ = m.forward_with_state(xd["u"][:, 50:], xd["delta"][:, 50:], xd["A"], xd["B"][:, 50:],
                                 xd["C"][:, 50:], xd["D"], h1)
    (torch.cat([o1, o2], 1) * xd["dout"]).sum().backward()
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], None, None, clamp=True)
    for k, name in GRADS:
        _close(name, xd[k].grad, r[name], torch.float32)


def test_extreme_delta_is_finite_and_matches(dev):
    """delta = 10 with A = -U(0, 0.1), fp16 (reference test_numerical_stability_extreme_values,
    tests/test_selective_scan.py:264-285)."""
    x = workloads.ssm_inputs(1, 512, 64, dtype=torch.float16, a_lo=0.0, a_hi=0.1, seed=9, dout=False)
    x["delta"] = torch.full_like(x["delta"], 10.0)
    out, h_last, _ = _run(x, dev, with_h=False, grads=False)
    assert torch.isfinite(out).all() and torch.isfinite(h_last).all()
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], None, clamp=True)
    _close("out", out, ro, torch.float16)


def test_exp_argument_clamp(dev):
    """delta*A = 120 is clamped to 88 before exp (mamba_cuda.py:65-70): with two steps the
    state stays finite (e^88 * tiny), where an unclamped fp32 exp(120) would be inf."""
    x = workloads.ssm_inputs(1, 2, 64, dtype=torch.float32, seed=9, dout=False)
    x["delta"] = torch.full_like(x["delta"], 10.0)
    x["A"][0, 0] = 12.0
    x["u"] = x["u"] * 1e-30
    out, h_last, _ = _run(x, dev, with_h=False, grads=False)
    assert torch.isfinite(out).all() and torch.isfinite(h_last).all()
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], None, clamp=True)
    assert np.isfinite(rh).all() and abs(rh[0, 0, 0]) > 1.0  # the clamp is live
    _close("out", out, ro, torch.float32)
    _close("h_last", h_last, rh, torch.float32)


def test_input_validation_on_device(dev):
    """reference tests/test_selective_scan.py:239-262: wrong h_prev N or batch -> RuntimeError."""
    x = {k: v.to(dev) for k, v in workloads.ssm_inputs(1, 64, 32, dtype=torch.float16, dout=False).items()}
    m = SelectiveScanCuda()
    with pytest.raises(RuntimeError):
        m(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], torch.randn(1, 32, 17, device=dev).half())
    with pytest.raises(RuntimeError):
        m(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], torch.randn(2, 32, 16, device=dev).half())


def test_no_grad_forward_keeps_nothing(dev):
    x = {k: v.to(dev) for k, v in workloads.ssm_inputs(2, 512, 512, dtype=torch.float16, dout=False).items()}
    m = SelectiveScanCuda()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    with torch.no_grad():
        out = m(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"])
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() - base <= out.numel() * out.element_size() + 4096


def _retained_after_forward(x, dev, lvl):
    """Device bytes a forward keeps alive for its backward (inputs excluded)."""
    leaves = {k: v.to(dev).requires_grad_(k != "dout") for k, v in x.items()}
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    out = SelectiveScanCuda(checkpoint_lvl=lvl)(leaves["u"], leaves["delta"], leaves["A"], leaves["B"],
                                                leaves["C"], leaves["D"])
    torch.cuda.synchronize()
    kept = torch.cuda.memory_allocated() - before - out.numel() * out.element_size()
    del out
    return kept


def test_config3_training_step_both_levels(dev):
    """Mamba-2.8B layer shape, fp16 (B=4, L=4096, D=5120): checkpoint levels 0 and 1 give
    bitwise-equal results, level 1 keeps nothing between forward and backward while level 0
    keeps the fp32 state every 16 steps, and both match the float64 oracle."""
    x = workloads.config_inputs("cfg3")
    B, L, D = 4, 4096, 5120
    kept0 = _retained_after_forward(x, dev, 0)
    kept1 = _retained_after_forward(x, dev, 1)
    assert kept0 >= B * ((L + 15) // 16) * D * 16 * 4
    assert kept1 < kept0 // 100
    print("case cfg3 level 0", flush=True)
    out0, _, g0 = _run(x, dev, with_h=False, lvl=0)
    print("case cfg3 level 1", flush=True)
    out1, _, g1 = _run(x, dev, with_h=False, lvl=1)
    assert torch.equal(out0, out1)
    for k in g0:
        assert torch.equal(g0[k], g1[k]), k
    del out1, g1
    print("case cfg3 oracle", flush=True)
    ro, _ = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], None, clamp=True)
    _close("out", out0, ro, torch.float16)
    del ro
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], None, None, clamp=True)
    for k, name in GRADS:
        _close(name, g0[k], r[name], torch.float16)


def test_config4a_streaming_long_sequence(dev):
    """fp32, B=1, L=131072, D=2048 fed as 32 chunks of 4096 through forward_with_state:
    h_last equals one full-length pass, and out/h_last match the float64 oracle on a
    256-channel slice (channels are independent in the forward)."""
    x = workloads.config_inputs("cfg4a", dout=False)
    xd = {k: v.to(dev) for k, v in x.items()}
    m = SelectiveScanCuda()
    with torch.no_grad():
        h = None
        outs = []
        for s0 in range(0, 131072, 4096):
            sl = slice(s0, s0 + 4096)
            o, h = m.forward_with_state(xd["u"][:, sl], xd["delta"][:, sl], xd["A"], xd["B"][:, sl],
                                        xd["C"][:, sl], xd["D"], h)
            outs.append(o[:, :, :256].cpu())
        full_out, full_h = m.forward_with_state(xd["u"], xd["delta"], xd["A"], xd["B"], xd["C"], xd["D"])
    torch.cuda.synchronize()
    # both passes may split L into segments at different points: agreement to the fp32 tolerance
    torch.testing.assert_close(h, full_h, **TOL[torch.float32])
    ro, rh = orc.ssm_fwd(x["u"][:, :, :256], x["delta"][:, :, :256], x["A"][:256], x["B"], x["C"],
                         x["D"][:256], None, clamp=True)
    _close("h_last", h[:, :256], rh, torch.float32)
    _close("out", torch.cat(outs, 1), ro, torch.float32)
    _close("out_full", full_out[:, :, :256], ro, torch.float32)


@pytest.mark.parametrize("shape", [(2, 0, 64), (0, 5, 64), (3, 5, 0), (1, 1, 1), (1, 17, 3)])
def test_empty_and_tiny_shapes(dev, shape):
    """Empty batch, sequence or channel axes and one-element shapes: outputs of the right shapes,
    h_last = h_prev and dh_prev = dh_last when L = 0, zero sums over an empty batch (dA, dD) or
    channel set (dB, dC), and the oracle wherever there is something to compute."""
    B, L, D = shape
    print(f"case empty/tiny shape={shape}", flush=True)
    x = workloads.ssm_inputs(B, L, D, dtype=torch.float32, h_prev=True, seed=B + L + D + 40)
    dhl = torch.randn(B, D, 16, generator=torch.Generator().manual_seed(41))
    out, h_last, g = _run(x, dev, with_h=True, dh_last=dhl)
    assert tuple(out.shape) == (B, L, D) and tuple(h_last.shape) == (B, D, 16)
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True)
    _close("out", out, ro, torch.float32)
    _close("h_last", h_last, rh, torch.float32)
    if L == 0:
        assert torch.equal(h_last.cpu(), x["h_prev"])
        assert torch.equal(g["h_prev"].cpu(), dhl)
    r = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], dhl, clamp=True)
    for k, name in GRADS + (("h_prev", "dh_prev"),):
        assert tuple(g[k].shape) == tuple(x[k].shape), name
        _close(name, g[k], r[name], torch.float32)
