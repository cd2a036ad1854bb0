"""Synthetic inputs for the benchmark configurations of the selective-scan path.

Recipes (seeded, generated in fp32 in the order u, delta, A, B, C, D, h_prev,
dout, then cast): "N(m,s)" is a normal with standard deviation s,
"U(a,b)" is a + (b-a)*rand.

  cfg0  fp32 B=1 L=1024 D=256;  u~N(0,1) delta~U(1e-3,1e-1) A=-U(0,0.1) B,C~N(0,1) D=1
  cfg1  fp16, as cfg0 plus h_prev~N(0,0.1) (B,D,16)
  cfg2  fp16 B=8 L=2048 D=1536; u~N(0,1) delta~U(1e-3,1e-1) A=-U(0.01,1) B,C~N(0,1)
        D~N(1,0.1) dout~N(0,1)                      (Mamba-130M layer shape)
  cfg3  fp16 B=4 L=4096 D=5120; as cfg2             (Mamba-2.8B layer shape)
  cfg4a fp32 B=1 L=131072 D=2048; as cfg2, streamed as 32 chunks of 4096
  cfg4b fp32 parallel scan over (4, 65536, 1024): a=0.9+0.1*rand, b~N(0,1)
"""
from __future__ import annotations

import torch

NSTATE = 16

CONFIGS = {
    "cfg0": dict(dtype=torch.float32, B=1, L=1024, D=256, a_lo=0.0, a_hi=0.1, d_mode="ones", h_prev=False),
    "cfg1": dict(dtype=torch.float16, B=1, L=1024, D=256, a_lo=0.0, a_hi=0.1, d_mode="ones", h_prev=True),
    "cfg2": dict(dtype=torch.float16, B=8, L=2048, D=1536, a_lo=0.01, a_hi=1.0, d_mode="normal", h_prev=False),
    "cfg3": dict(dtype=torch.float16, B=4, L=4096, D=5120, a_lo=0.01, a_hi=1.0, d_mode="normal", h_prev=False),
    "cfg4a": dict(dtype=torch.float32, B=1, L=131072, D=2048, a_lo=0.01, a_hi=1.0, d_mode="normal", h_prev=False),
}


def ssm_inputs(B, L, D, *, dtype=torch.float32, a_lo=0.01, a_hi=1.0, d_mode="normal", h_prev=False,
               dout=True, seed=0, device="cpu", gen_device="cpu", nstate=NSTATE):
    """Seeded selective-scan inputs (state count `nstate`). Returns a dict of tensors on `device`."""
    g = torch.Generator(device=gen_device).manual_seed(seed)
    kw = dict(generator=g, device=gen_device, dtype=torch.float32)
    r = {}
    r["u"] = torch.randn(B, L, D, **kw)
    r["delta"] = 1e-3 + (1e-1 - 1e-3) * torch.rand(B, L, D, **kw)
    r["A"] = -(a_lo + (a_hi - a_lo) * torch.rand(D, nstate, **kw))
    r["B"] = torch.randn(B, L, nstate, **kw)
    r["C"] = torch.randn(B, L, nstate, **kw)
    r["D"] = torch.ones(D, device=gen_device) if d_mode == "ones" else 1.0 + 0.1 * torch.randn(D, **kw)
    if h_prev:
        r["h_prev"] = 0.1 * torch.randn(B, D, nstate, **kw)
    if dout:
        r["dout"] = torch.randn(B, L, D, **kw)
    return {k: v.to(device=device, dtype=dtype) for k, v in r.items()}


def config_inputs(name, *, seed=0, device="cpu", gen_device="cpu", dout=True):
    c = dict(CONFIGS[name])
    return ssm_inputs(c.pop("B"), c.pop("L"), c.pop("D"), seed=seed, device=device, gen_device=gen_device,
                      dout=dout, **c)


def pscan_inputs(shape=(4, 65536, 1024), *, dtype=torch.float32, seed=0, device="cpu", gen_device="cpu"):
    """a = 0.9 + 0.1*rand, b ~ N(0,1) of `shape` (cfg4b)."""
    g = torch.Generator(device=gen_device).manual_seed(seed)
    a = 0.9 + 0.1 * torch.rand(shape, generator=g, device=gen_device)
    b = torch.randn(shape, generator=g, device=gen_device)
    return a.to(device=device, dtype=dtype), b.to(device=device, dtype=dtype)


def algorithmic_bytes(B, L, D, elem_bytes, *, fwd=True, bwd=True, state_io=False, nstate=NSTATE):
    """Compulsory HBM bytes of the fused path (inputs read once, outputs written once).

    fwd = s*(3BLD + 2BLN + DN + D)       (u, delta in; out; B, C; A; D)
    bwd = s*(5BLD + 4BLN + 2DN + 2D)     (u, delta, dout in; du, ddelta out; B, C in; dB, dC out; A, dA; D, dD)
    state_io adds s*2BDN per direction (h_prev in / h_last out, dh_last in / dh_prev out)."""
    N = nstate
    s = elem_bytes
    n = 0
    if fwd:
        n += s * (3 * B * L * D + 2 * B * L * N + D * N + D)
    if bwd:
        n += s * (5 * B * L * D + 4 * B * L * N + 2 * D * N + 2 * D)
    if state_io:
        n += s * 2 * B * D * N * (int(fwd) + int(bwd))
    return n
