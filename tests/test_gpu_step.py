"""GPU parity of the decode step (L = 1 with a carried state) against the float64 oracle.

Tolerances as in test_gpu_ssm.py: fp32 rtol 1e-3 / atol 1e-4, fp16 rtol 1e-2 / atol 1e-2.
"""
import numpy as np
import pytest
import torch

from mamba_windows_cuda import SelectiveScanCuda, workloads
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.float16: dict(rtol=1e-2, atol=1e-2),
       torch.bfloat16: dict(rtol=2e-2, atol=2e-2)}


def _close(name, got, ref, dtype):
    np.testing.assert_allclose(got.detach().cpu().double().numpy(), ref, err_msg=name, **TOL[dtype])


def _step_inputs(Bsz, D, dtype, seed):
    x = workloads.ssm_inputs(Bsz, 1, D, dtype=torch.float32, h_prev=True, dout=False, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    x["h_prev"] = torch.randn(Bsz, D, 16, generator=g)
    x["z"] = torch.randn(Bsz, 1, D, generator=g)
    x["delta_bias"] = 0.5 * torch.randn(D, generator=g)
    return {k: v.to(dtype) for k, v in x.items()}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 70), (8, 1536), (3, 2100)])
@pytest.mark.parametrize("xf", [False, True])
def test_step_matches_oracle(dev, dtype, shape, xf):
    Bsz, D = shape
    print(f"case step shape={shape} dtype={dtype} xf={xf}", flush=True)
    x = _step_inputs(Bsz, D, dtype, seed=Bsz + D)
    xd = {k: v.to(dev) for k, v in x.items()}
    kw = dict(z=xd["z"][:, 0], delta_bias=xd["delta_bias"], delta_softplus=True) if xf else {}
    with torch.no_grad():
        y, h = SelectiveScanCuda().step(xd["u"][:, 0], xd["delta"][:, 0], xd["A"], xd["B"][:, 0], xd["C"][:, 0],
                                        xd["D"], xd["h_prev"], **kw)
    okw = dict(delta_bias=x["delta_bias"], delta_softplus=True, z=x["z"]) if xf else {}
    ro, rh, _ = orc.ssm_fwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], clamp=True, **okw)
    _close("out", y, ro[:, 0], dtype)
    _close("h_new", h, rh, dtype)


def test_chained_steps_equal_forward(dev):
    """K decode steps reproduce one forward_with_state pass over K steps (out rows and state)."""
    Bsz, L, D = 4, 24, 300
    x = workloads.ssm_inputs(Bsz, L, D, dtype=torch.float32, h_prev=True, dout=False, seed=31)
    xd = {k: v.to(dev) for k, v in x.items()}
    m = SelectiveScanCuda()
    with torch.no_grad():
        full, h_full = m.forward_with_state(xd["u"], xd["delta"], xd["A"], xd["B"], xd["C"], xd["D"], xd["h_prev"])
        h = xd["h_prev"].clone()
        for t in range(L):
            y, _ = m.step(xd["u"][:, t], xd["delta"][:, t], xd["A"], xd["B"][:, t], xd["C"][:, t], xd["D"], h,
                          out_state=h)  # in place
            torch.testing.assert_close(y, full[:, t], **TOL[torch.float32])
    torch.testing.assert_close(h, h_full, **TOL[torch.float32])


def test_in_place_equals_out_of_place(dev):
    x = _step_inputs(5, 257, torch.float16, seed=3)
    xd = {k: v.to(dev) for k, v in x.items()}
    m = SelectiveScanCuda()
    args = (xd["u"][:, 0], xd["delta"][:, 0], xd["A"], xd["B"][:, 0], xd["C"][:, 0], xd["D"])
    with torch.no_grad():
        y1, h1 = m.step(*args, xd["h_prev"])
        h = xd["h_prev"].clone()
        v0 = h._version
        y2, h2 = m.step(*args, h, out_state=h)
    assert h2.data_ptr() == h.data_ptr()
    assert h._version > v0  # the in-place write is visible to autograd's version check
    assert torch.equal(y1, y2) and torch.equal(h1, h2)


def test_step_is_inference_only(dev):
    x = _step_inputs(2, 16, torch.float32, seed=5)
    xd = {k: v.to(dev) for k, v in x.items()}
    u = xd["u"][:, 0].clone().requires_grad_(True)
    with pytest.raises(RuntimeError, match="inference-only"):
        SelectiveScanCuda().step(u, xd["delta"][:, 0], xd["A"], xd["B"][:, 0], xd["C"][:, 0], xd["D"], xd["h_prev"])


def test_step_graph_replay(dev):
    """Decode steps captured once in a HIP graph and replayed match eager steps (state in place)."""
    x = _step_inputs(4, 300, torch.float32, seed=12)
    xd = {k: v.to(dev) for k, v in x.items()}
    m = SelectiveScanCuda()
    args = (xd["u"][:, 0].contiguous(), xd["delta"][:, 0].contiguous(), xd["A"], xd["B"][:, 0].contiguous(),
            xd["C"][:, 0].contiguous(), xd["D"])
    with torch.no_grad():
        h_eager = xd["h_prev"].clone()
        for _ in range(5):
            y_eager, _ = m.step(*args, h_eager, out_state=h_eager)
        h = xd["h_prev"].clone()
        m.step(*args, h, out_state=h)  # warm the allocator outside the capture
        h.copy_(xd["h_prev"])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y, _ = m.step(*args, h, out_state=h)
        for r in range(4):  # the capture itself ran nothing; 4 replays + 1 eager step = 5 steps
            graph.replay()
            torch.cuda.synchronize()
        y2, _ = m.step(*args, h, out_state=h)
        torch.cuda.synchronize()
    assert torch.equal(h, h_eager)
    assert torch.equal(y2, y_eager)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_step_misaligned_state(dev, dtype):
    """The step moves a lane's states as one 16-byte vector: a state view that starts off a 16-byte
    boundary is copied by the Python layer (same result as an aligned one), and an out_state view that
    does is refused with RuntimeError."""
    Bsz, D = 3, 130
    x = _step_inputs(Bsz, D, dtype, seed=5)
    xd = {k: v.to(dev) for k, v in x.items()}
    m = SelectiveScanCuda()
    args = (xd["u"][:, 0], xd["delta"][:, 0], xd["A"], xd["B"][:, 0], xd["C"][:, 0], xd["D"])
    # the same state, starting one element (4 or 2 bytes) past a 16-byte boundary
    buf = torch.zeros(Bsz * D * 16 + 1, dtype=dtype, device=dev)
    h_off = buf[1:].view(Bsz, D, 16)
    h_off.copy_(xd["h_prev"])
    assert h_off.data_ptr() % 16 != 0
    with torch.no_grad():
        y_ref, h_ref = m.step(*args, xd["h_prev"])
        y, h = m.step(*args, h_off)
        assert torch.equal(y, y_ref) and torch.equal(h, h_ref)
        with pytest.raises(RuntimeError, match="16-byte-aligned"):
            m.step(*args, xd["h_prev"], out_state=h_off)
