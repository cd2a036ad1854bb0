"""The C++ host path (torch.ops.mwc.ssm_scan, csrc/torch_ops.cpp), which SelectiveScanCuda and
FusedSelectiveScan call, against the Python host path (SelectiveScanCudaFunction over ops.py and
ctypes): both enqueue the same kernels with the same launch plans, so out, h_last and every gradient
must agree bitwise, for every combination of h_prev, the fused transforms, checkpoint level and
storage dtype. Also: the argument checks give the reference's messages on device tensors, and a call
that needs no gradient keeps nothing."""
import pytest
import torch

from mamba_windows_cuda import SelectiveScanCuda, workloads
from mamba_windows_cuda.mamba_cuda import SelectiveScanCudaFunction, _ssm_scan

pytestmark = pytest.mark.gpu

NAMES = ("u", "delta", "A", "B", "C", "D")


def _leaves(x, dev, keys):
    return {k: x[k].to(dev).requires_grad_(True) for k in keys}


def _step(fn, x, dev, *, with_h, gated, biased, softplus, lvl, dh_last):
    keys = NAMES + (("h_prev",) if with_h else ())
    lv = _leaves(x, dev, keys)
    extra = {}
    if gated:
        extra["z"] = x["z"].to(dev).requires_grad_(True)
    if biased:
        extra["delta_bias"] = x["delta_bias"].to(dev).requires_grad_(True)
    out, h_last = fn(*(lv[k] for k in NAMES), lv.get("h_prev"), lvl, extra.get("z"), extra.get("delta_bias"),
                     softplus)
    loss = (out.float() * x["dout"].to(dev).float()).sum()
    if dh_last:
        loss = loss + (h_last.float() * x["dh_last"].to(dev).float()).sum()
    loss.backward()
    torch.cuda.synchronize()
    grads = {k: t.grad for k, t in {**lv, **extra}.items()}
    return out.detach(), h_last.detach(), grads


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("with_h,gated,biased,softplus,lvl,dh_last", [
    (False, False, False, False, 0, False),
    (True, False, False, False, 0, True),
    (True, False, False, False, 1, True),
    (False, True, True, True, 0, False),
    (True, True, True, True, 1, True),
    (False, False, True, False, 1, False),
], ids=["plain", "h_prev", "h_prev_lvl1", "xf", "xf_h_lvl1", "bias_lvl1"])
def test_cpp_path_equals_python_path_bitwise(dev, dtype, with_h, gated, biased, softplus, lvl, dh_last):
    print(f"case torch op vs python {dtype} h={with_h} z={gated} bias={biased} sp={softplus} lvl={lvl}",
          flush=True)
    B, L, D = 2, 300, 96
    x = workloads.ssm_inputs(B, L, D, dtype=dtype, h_prev=True, seed=17)
    g = torch.Generator().manual_seed(5)
    x["z"] = torch.randn(B, L, D, generator=g).to(dtype)
    x["delta_bias"] = (0.1 * torch.randn(D, generator=g)).to(dtype)
    x["dh_last"] = torch.randn(B, D, 16, generator=g).to(dtype)
    kw = dict(with_h=with_h, gated=gated, biased=biased, softplus=softplus, lvl=lvl, dh_last=dh_last)
    o1, h1, g1 = _step(_ssm_scan, x, dev, **kw)
    o2, h2, g2 = _step(SelectiveScanCudaFunction.apply, x, dev, **kw)
    assert torch.equal(o1, o2) and torch.equal(h1, h2)
    assert g1.keys() == g2.keys()
    for k in g1:
        assert g1[k] is not None and torch.equal(g1[k], g2[k]), k


@pytest.mark.parametrize("mutate,msg", [
    (lambda x: x.update(A=torch.randn(3, 15)), "Only N=16"),
    (lambda x: x.update(A=torch.randn(3, 32)), "B_ssm shape mismatch"),
    (lambda x: x.update(u=x["u"].double()), "float32/float16"),
    (lambda x: x.update(delta=x["delta"].half()), "delta dtype must match"),
    (lambda x: x.update(u=x["u"][0]), "u must be 3D"),
    (lambda x: x.update(B=torch.randn(2, 4, 16)), "B_ssm shape mismatch"),
    (lambda x: x.update(D=torch.ones(4)), "D_ssm shape mismatch"),
    (lambda x: x.update(C=torch.randn(2, 16, 5).transpose(1, 2)), "C_ssm must be contiguous"),
    (lambda x: x.update(h_prev=torch.randn(2, 3, 17)), "h_prev shape must be"),
    (lambda x: x.update(h_prev=torch.randn(3, 3, 16)), "h_prev shape must be"),
    (lambda x: x.update(h_prev=torch.randn(2, 3, 16).half()), "h_prev dtype"),
    (lambda x: x.update(z=torch.randn(2, 5, 4)), r"z shape must be \(2, 5, 3\)"),
    (lambda x: x.update(delta_bias=torch.randn(4)), r"delta_bias shape must be \(3,\)"),
    (lambda x: x.update(lvl=2), "checkpoint_lvl must be 0 or 1"),
])
def test_operator_argument_checks(dev, mutate, msg):
    """The reference's TORCH_CHECK contract (mamba_cuda.py:281-326) on device tensors, raised before any
    work is queued."""
    x = dict(u=torch.randn(2, 5, 3), delta=torch.rand(2, 5, 3), A=-torch.rand(3, 16), B=torch.randn(2, 5, 16),
             C=torch.randn(2, 5, 16), D=torch.ones(3), h_prev=None, z=None, delta_bias=None, lvl=0)
    mutate(x)
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in x.items()}
    with pytest.raises(RuntimeError, match=msg):
        _ssm_scan(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["h_prev"], d["lvl"], d["z"],
                  d["delta_bias"], False)


def test_operator_without_gradients_keeps_nothing(dev):
    x = {k: v.to(dev) for k, v in workloads.ssm_inputs(1, 100, 64, seed=3).items()}
    m = SelectiveScanCuda()
    ref = m(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"])
    assert ref.grad_fn is None
    with torch.inference_mode():
        out = m(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"])
    lv = {k: x[k].clone().requires_grad_(True) for k in NAMES}
    with torch.no_grad():
        out2 = m(*(lv[k] for k in NAMES))
    assert out2.grad_fn is None
    assert torch.equal(out, ref) and torch.equal(out2, ref)


def test_operator_gradient_from_h_last_only(dev):
    """A loss on h_last alone gives no dout: the backward treats it as zeros (and vice versa)."""
    x = workloads.ssm_inputs(2, 70, 40, h_prev=True, seed=9)
    res = []
    for fn in (_ssm_scan, SelectiveScanCudaFunction.apply):
        lv = {k: x[k].to(dev).requires_grad_(True) for k in NAMES + ("h_prev",)}
        out, h_last = fn(*(lv[k] for k in NAMES), lv["h_prev"], 0, None, None, False)
        h_last.sum().backward()
        torch.cuda.synchronize()
        res.append({k: t.grad for k, t in lv.items()})
    for k in res[0]:
        assert torch.equal(res[0][k], res[1][k]), k


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("xf", [False, True], ids=["plain", "xf"])
def test_step_operator_equals_python_step(dev, dtype, xf):
    """SelectiveScanCuda.step (torch.ops.mwc.ssm_step) against ops.ssm_step: out and h_new bitwise, out of
    place and in place, and with A / h that are not 16-byte aligned (both paths copy them first)."""
    from mamba_windows_cuda import ops

    print(f"case step operator vs python {dtype} xf={xf}", flush=True)
    Bsz, D, N = 5, 200, 16
    x = workloads.ssm_inputs(Bsz, 1, D, dtype=dtype, h_prev=True, seed=23)
    g = torch.Generator().manual_seed(2)
    kw = {}
    if xf:
        kw = dict(z=torch.randn(Bsz, D, generator=g).to(dtype).to(dev),
                  delta_bias=(0.1 * torch.randn(D, generator=g)).to(dtype).to(dev), delta_softplus=True)
    args = [x["u"][:, 0].to(dev), x["delta"][:, 0].to(dev), x["A"].to(dev), x["B"][:, 0].to(dev),
            x["C"][:, 0].to(dev), x["D"].to(dev)]
    h = x["h_prev"].to(dev)
    m = SelectiveScanCuda()
    y1, h1 = m.step(*args, h, **kw)
    y2, h2 = ops.ssm_step(*args, h, **kw)
    assert torch.equal(y1, y2) and torch.equal(h1, h2)
    hc = h.clone()
    y3, h3 = m.step(*args, hc, out_state=hc, **kw)
    assert h3.data_ptr() == hc.data_ptr() and torch.equal(y3, y1) and torch.equal(hc, h1)
    # misaligned A and h: views one element into a larger buffer
    A_buf = torch.empty(D * N + 1, dtype=dtype, device=dev)
    A_mis = A_buf[1:].view(D, N)
    A_mis.copy_(args[2])
    h_buf = torch.empty(Bsz * D * N + 1, dtype=dtype, device=dev)
    h_mis = h_buf[1:].view(Bsz, D, N)
    h_mis.copy_(h)
    y4, h4 = m.step(args[0], args[1], A_mis, *args[3:], h_mis, **kw)
    torch.cuda.synchronize()
    assert torch.equal(y4, y1) and torch.equal(h4, h1)


def test_operands_on_another_device_are_refused(dev):
    """Every operand a kernel reads must be on u's device: a host dout, dh_last, checkpoint or
    out_state raises RuntimeError before anything is enqueued."""
    from mamba_windows_cuda import ops

    x = {k: v.to(dev) for k, v in workloads.ssm_inputs(1, 40, 32, h_prev=True, seed=4).items()}
    _, _, h_last, ckpt = ops.ssm_forward_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], want_ckpt=True)
    args = (x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"])
    with pytest.raises(RuntimeError, match="dout must be on the same device"):
        ops.ssm_backward(*args, x["dout"].cpu(), ckpt)
    with pytest.raises(RuntimeError, match="dh_last must be on the same device"):
        ops.ssm_backward(*args, x["dout"], ckpt, h_last.cpu())
    with pytest.raises(RuntimeError, match="ckpt must be on the same device"):
        ops.ssm_backward(*args, x["dout"], ckpt.cpu())
    step_args = (x["u"][:, 0], x["delta"][:, 0], x["A"], x["B"][:, 0], x["C"][:, 0], x["D"], x["h_prev"])
    with pytest.raises(RuntimeError, match="out_state must be"):
        SelectiveScanCuda().step(*step_args, out_state=torch.zeros(1, 32, 16))
    torch.cuda.synchronize()


@pytest.mark.parametrize("lvl", [0, 1])
def test_strided_views_equal_contiguous_copies(dev, lvl):
    """Inputs that are views with a contiguous last dimension but other strides (an L-slice with B > 1,
    a D-slice of a wider tensor, A as the first 16 columns of a (D, 32) tensor, a B-slice of h_prev):
    the operator copies them to contiguous tensors first, as the reference does
    (mamba_cuda.py:1197-1199), so outputs and the gradients reaching the base tensors equal those of
    contiguous copies, bitwise."""
    print(f"case strided views lvl={lvl}", flush=True)
    g = torch.Generator().manual_seed(12)
    Bsz, L, D, N = 3, 200, 96, 16
    base = {"u": torch.randn(Bsz, L + 50, D + 8, generator=g),
            "delta": 0.01 + 0.09 * torch.rand(Bsz, L + 50, D + 8, generator=g),
            "A": -torch.rand(D, 2 * N, generator=g), "B": torch.randn(Bsz, L + 50, N, generator=g),
            "C": torch.randn(Bsz, L + 50, N, generator=g), "D": torch.randn(D, generator=g),
            "h_prev": torch.randn(Bsz + 1, D, N, generator=g)}
    dout = torch.randn(Bsz, L, D, generator=g).to(dev)

    def views(t):
        return (t["u"][:, 20:20 + L, 4:4 + D], t["delta"][:, 20:20 + L, 4:4 + D], t["A"][:, :N],
                t["B"][:, 20:20 + L], t["C"][:, 20:20 + L], t["D"], t["h_prev"][1:])

    res = []
    for contiguous in (False, True):
        leaves = {k: v.to(dev).requires_grad_(True) for k, v in base.items()}
        args = views(leaves)
        assert contiguous or not all(a.is_contiguous() for a in args)
        if contiguous:
            args = tuple(a.contiguous() for a in args)
        out, h_last = SelectiveScanCuda(checkpoint_lvl=lvl).forward_with_state(*args)
        ((out * dout).sum() + h_last.sum()).backward()
        torch.cuda.synchronize()
        res.append((out.detach(), h_last.detach(), {k: t.grad for k, t in leaves.items()}))
    (o1, h1, g1), (o2, h2, g2) = res
    assert torch.equal(o1, o2) and torch.equal(h1, h2)
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k
