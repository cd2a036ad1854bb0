"""Opt-in randomized sweeps of parallel_scan_fn (forward and adjoint) and of the decode step against
the float64 oracle. MWC_SWEEP_CASES=N runs N seeded cases of each (default 0: nothing is
collected); the cases are the same on every run.

* parallel_scan_fn: 3-D (B, L, C) and 4-D (B, D, L, N) inputs up to 3,000 steps, fp32/fp16/bf16,
  a ~ U(0.8, 1.0); tolerance rtol plus atol scaled by the result's largest magnitude (the scan's
  outputs grow with L).
* decode step: every state count, dtype and transform combination (bias, softplus, z gate) at L=1,
  against the oracle's forward over one step.
"""
import os
import random

import numpy as np
import pytest
import torch

from mamba_windows_cuda import SelectiveScanCuda, parallel_scan_fn, workloads
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
NCASES = int(os.environ.get("MWC_SWEEP_CASES", "0"))
TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.float16: dict(rtol=1e-2, atol=1e-2),
       torch.bfloat16: dict(rtol=2e-2, atol=2e-2)}


def _scaled(got, ref, tol):
    np.testing.assert_allclose(got.detach().cpu().double().numpy(), ref, rtol=tol["rtol"],
                               atol=tol["atol"] * max(1.0, float(np.abs(ref).max())))


if NCASES > 0:  # opt-in

    @pytest.mark.parametrize("idx", range(NCASES))
    def test_pscan_sweep(dev, idx):
        r = random.Random(777 + idx)
        dtype = r.choice((torch.float32, torch.float16, torch.bfloat16))
        if r.random() < 0.5:
            shape = (r.randint(1, 3), r.randint(1, 40), r.randint(1, 700), r.choice((1, 4, 16, 33)))
        else:
            shape = (r.randint(1, 3), r.randint(1, 3000), r.randint(1, 300))
        print(f"case pscan idx={idx} shape={shape} dtype={dtype}", flush=True)
        g = torch.Generator().manual_seed(idx)
        A = (0.8 + 0.2 * torch.rand(shape, generator=g)).to(dtype)
        X = torch.randn(shape, generator=g).to(dtype)
        dH = torch.randn(shape, generator=g).to(dtype)
        Ad, Xd = A.to(dev).requires_grad_(True), X.to(dev).requires_grad_(True)
        H = parallel_scan_fn(Ad, Xd)
        H.backward(dH.to(dev))
        torch.cuda.synchronize()
        Hr = orc.pscan_fwd(A, X)
        dAr, dXr = orc.pscan_bwd(A, Hr, dH)
        tol = dict(TOL[dtype], rtol=1e-4) if dtype == torch.float32 else TOL[dtype]
        _scaled(H, Hr, tol)
        _scaled(Xd.grad, dXr, tol)
        _scaled(Ad.grad, dAr, tol)


    @pytest.mark.parametrize("idx", range(NCASES))
    def test_step_sweep(dev, idx):
        r = random.Random(555 + idx)
        n = r.choice((8, 16, 32, 64))
        dtype = r.choice((torch.float32, torch.float16, torch.bfloat16))
        Bsz, D = r.randint(1, 70), r.randint(1, 900)
        sp, bias, gate = r.random() < 0.4, r.random() < 0.4, r.random() < 0.4
        print(f"case step idx={idx} B={Bsz} D={D} N={n} dtype={dtype} softplus={sp} bias={bias} gate={gate}",
              flush=True)
        x = workloads.ssm_inputs(Bsz, 1, D, dtype=torch.float32, h_prev=True, seed=idx, nstate=n)
        g = torch.Generator().manual_seed(idx + 1)
        db = (0.05 * torch.rand(D, generator=g)).to(dtype) if bias else None
        z = torch.randn(Bsz, D, generator=g).to(dtype) if gate else None
        x = {k: v.to(dtype) for k, v in x.items()}
        y, h = SelectiveScanCuda().step(x["u"][:, 0].to(dev), x["delta"][:, 0].to(dev), x["A"].to(dev),
                                        x["B"][:, 0].to(dev), x["C"][:, 0].to(dev), x["D"].to(dev),
                                        x["h_prev"].to(dev), z=None if z is None else z.to(dev),
                                        delta_bias=None if db is None else db.to(dev), delta_softplus=sp)
        torch.cuda.synchronize()
        ro, rh, _ = orc.ssm_fwd_xf(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"], delta_bias=db,
                                   delta_softplus=sp, z=None if z is None else z[:, None], clamp=True)
        np.testing.assert_allclose(y.cpu().double().numpy(), ro[:, 0], **TOL[dtype])
        np.testing.assert_allclose(h.cpu().double().numpy(), rh, **TOL[dtype])
