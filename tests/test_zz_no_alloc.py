"""mwc_ssm_fwd_noalloc (the forward that allocates nothing, its segment carries in a static
per-device scratch array) against mwc_ssm_fwd_ex with a caller workspace, through the C ABI:
bitwise-equal outputs on calls in a row, each smaller than the one before, with L split into segments
so that the scratch is used -- the planner's own plan at a small-problem shape, forced plans at one and
two states per lane, N=8 at two states per lane; and the size limit."""
import ctypes

import pytest
import torch

from mamba_windows_cuda import _lib, ops, workloads


def _p(t):
    return None if t is None else t.data_ptr()


def _fwd_both(dev, B, L, D, dtype, *, xf, seed, n=16):
    x = {k: v.to(dev) for k, v in workloads.ssm_inputs(B, L, D, dtype=dtype, h_prev=True, dout=False,
                                                       seed=seed, nstate=n).items()}
    bias = (0.3 * torch.randn(D, generator=torch.Generator().manual_seed(seed))).to(dtype).to(dev) if xf else None
    z = torch.randn(B, L, D, generator=torch.Generator().manual_seed(seed + 1)).to(dtype).to(dev) if xf else None
    L_ = _lib.lib()
    nbytes = L_.mwc_ssm_fwd_workspace_size(B, L, D, n)
    assert 0 < nbytes <= _lib.NOALLOC_SCRATCH_BYTES  # L is split: the scratch is in use
    nck = L_.mwc_ssm_ckpt_count(L)
    results = []
    for which in ("ex", "noalloc"):
        out = torch.full_like(x["u"], float("nan"))
        out_z = torch.full_like(x["u"], float("nan")) if xf else None
        h_last = torch.full((B, D, n), float("nan"), dtype=dtype, device=dev)
        ckpt = torch.full((B, nck, D, n), float("nan"), dtype=torch.float32, device=dev)
        args = (ops._dtype_code(x["u"]), x["u"].data_ptr(), x["delta"].data_ptr(), x["A"].data_ptr(),
                x["B"].data_ptr(), x["C"].data_ptr(), x["D"].data_ptr(), x["h_prev"].data_ptr(),
                _p(bias), int(xf), _p(z), out.data_ptr(), _p(out_z), h_last.data_ptr(),
                ckpt.data_ptr(), B, L, D, n)
        if which == "ex":
            ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            st = L_.mwc_ssm_fwd_ex(*args, ws.data_ptr(), nbytes, ops._stream(x["u"].device))
        else:
            st = L_.mwc_ssm_fwd_noalloc(*args, ops._stream(x["u"].device))
        _lib.check(st, which)
        torch.cuda.synchronize()
        results.append((out, out_z, h_last, ckpt))
    return results


# (B, L, D, N, dtype, fused transforms, seed, forced plan): each smaller than the one before
CASES = (
    (8, 2048, 192, 16, torch.float16, False, 64, None),            # the planner's plan (16 segments)
    (4, 600, 700, 16, torch.float16, True, 63, ("3", "2")),        # B*D >= 2048: two states per lane
    (3, 500, 800, 8, torch.bfloat16, False, 65, ("3", "2")),       # N=8 at two states per lane
    (3, 700, 500, 16, torch.float16, False, 61, ("3", "2")),       # one state per lane
    (2, 300, 130, 16, torch.float32, True, 62, ("3", "2")),
)


@pytest.mark.gpu
def test_noalloc_forward_matches_workspace_forward(dev, monkeypatch):
    # calls in a row on the same GPU, each bitwise equal to the workspace entry point's results
    for B, L, D, n, dtype, xf, seed, forced in CASES:
        print(f"case noalloc B={B} L={L} D={D} N={n} dtype={dtype} transforms={xf} plan={forced}", flush=True)
        for var, val in zip(("MWC_NSEG", "MWC_CFOLD"), forced or (None, None)):
            if val is None:
                monkeypatch.delenv(var, raising=False)
            else:
                monkeypatch.setenv(var, val)
        (o1, z1, h1, c1), (o2, z2, h2, c2) = _fwd_both(dev, B, L, D, dtype, xf=xf, seed=seed, n=n)
        assert torch.isfinite(o1).all() and torch.isfinite(h1).all() and torch.isfinite(c1).all()
        assert torch.equal(o1, o2) and torch.equal(h1, h2) and torch.equal(c1, c2)
        if xf:
            assert torch.isfinite(z1).all() and torch.equal(z1, z2)


def test_noalloc_forward_rejects_sizes_beyond_its_scratch(monkeypatch):
    """Carries beyond MWC_NOALLOC_SCRATCH_BYTES: MWC_ERR_UNSUPPORTED before anything is enqueued (the
    pointers are never dereferenced, so this runs without a GPU)."""
    monkeypatch.setenv("MWC_NSEG", "16")
    monkeypatch.setenv("MWC_CFOLD", "4")
    L_ = _lib.lib()
    B, L, D = 64, 8192, 8192
    assert L_.mwc_ssm_fwd_workspace_size(B, L, D, 16) > _lib.NOALLOC_SCRATCH_BYTES
    fake = ctypes.c_void_p(256)
    st = L_.mwc_ssm_fwd_noalloc(1, fake, fake, fake, fake, fake, fake, None, None, 0, None, fake, None, None, None,
                                B, L, D, 16, None)
    assert st == 2 and b"scratch" in L_.mwc_last_error()
