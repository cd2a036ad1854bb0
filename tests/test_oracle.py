"""Pins for the float64 C oracle (CPU only).

Each check is independent of the oracle's own formula: torch autograd
through a sequential float64 restatement of ``selective_scan_ref``
(mamba_cuda.py:875-946), finite differences, the reference tests' cumsum
closed form (tests/test_selective_scan.py:8-36), and special cases whose
answer the mathematics fixes.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from oracle import torch_ref

F64 = torch.float64


def _inputs(bsz, L, dm, n=16, seed=0, a_lo=0.01, a_hi=1.0, h_prev=True):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(bsz, L, dm, generator=g, dtype=F64)
    delta = 1e-3 + (1e-1 - 1e-3) * torch.rand(bsz, L, dm, generator=g, dtype=F64)
    A = -(a_lo + (a_hi - a_lo) * torch.rand(dm, n, generator=g, dtype=F64))
    B = torch.randn(bsz, L, n, generator=g, dtype=F64)
    C = torch.randn(bsz, L, n, generator=g, dtype=F64)
    D = 1.0 + 0.1 * torch.randn(dm, generator=g, dtype=F64)
    hp = 0.1 * torch.randn(bsz, dm, n, generator=g, dtype=F64) if h_prev else None
    return u, delta, A, B, C, D, hp


@pytest.mark.parametrize("shape", [(1, 7, 5, 16), (2, 33, 19, 16), (3, 64, 70, 4), (1, 1, 3, 16)])
@pytest.mark.parametrize("with_h", [False, True])
def test_fwd_matches_sequential_torch(shape, with_h):
    u, delta, A, B, C, D, hp = _inputs(*shape, seed=sum(shape), h_prev=with_h)
    out, hl = orc.ssm_fwd(u, delta, A, B, C, D, hp)
    ro, rh = torch_ref.selective_scan_seq(u, delta, A, B, C, D, hp)
    np.testing.assert_allclose(out, ro.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(hl, rh.numpy(), rtol=1e-12, atol=1e-12)
    vo, vh = torch_ref.selective_scan_vectorized(u, delta, A, B, C, D, hp)
    np.testing.assert_allclose(out, vo.numpy(), rtol=1e-12, atol=1e-12)


def test_fwd_matches_closed_form():
    # the reference tests' own oracle: benign |A*cumsum(delta)|
    g = torch.Generator().manual_seed(3)
    bsz, L, dm, n = 2, 256, 24, 16
    u = 0.1 * torch.randn(bsz, L, dm, generator=g, dtype=F64)
    delta = torch.full((bsz, L, dm), 0.01, dtype=F64)
    A = -0.1 * torch.rand(dm, n, generator=g, dtype=F64)
    B = 0.1 * torch.randn(bsz, L, n, generator=g, dtype=F64)
    C = 0.1 * torch.randn(bsz, L, n, generator=g, dtype=F64)
    D = torch.full((dm,), 0.1, dtype=F64)
    hp = torch.randn(bsz, dm, n, generator=g, dtype=F64)
    out, hl = orc.ssm_fwd(u, delta, A, B, C, D, hp)
    co, ch = torch_ref.selective_scan_closed(u, delta, A, B, C, D, hp)
    np.testing.assert_allclose(out, co.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(hl, ch.numpy(), rtol=1e-9, atol=1e-11)


def test_fwd_special_cases():
    u, delta, A, B, C, D, hp = _inputs(2, 40, 9, seed=5)
    # A = 0: h_t = h_prev + cumsum(delta*u*B)
    A0 = torch.zeros_like(A)
    out, hl = orc.ssm_fwd(u, delta, A0, B, C, D, hp)
    h = hp.unsqueeze(2) + torch.cumsum((delta * u).unsqueeze(-1) * B.unsqueeze(2), dim=1).transpose(1, 2)
    # h: (B,D,L,N)
    y = (h * C.unsqueeze(1)).sum(-1).transpose(1, 2) + D * u
    np.testing.assert_allclose(out, y.numpy(), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(hl, h[:, :, -1].numpy(), rtol=1e-11, atol=1e-11)
    # delta = 0: state constant, y = C.h_prev + D*u
    out, hl = orc.ssm_fwd(u, torch.zeros_like(delta), A, B, C, D, hp)
    y = torch.einsum("bdn,bln->bld", hp, C) + D * u
    np.testing.assert_allclose(out, y.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(hl, hp.numpy(), rtol=0, atol=0)
    # B = 0: h_t = exp(A*S_t) h_prev
    out, hl = orc.ssm_fwd(u, delta, A, torch.zeros_like(B), C, D, hp)
    S = torch.cumsum(delta, dim=1)  # (B,L,D)
    ht = torch.exp(S.unsqueeze(-1) * A) * hp.unsqueeze(1)  # (B,L,D,N)
    np.testing.assert_allclose(hl, ht[:, -1].numpy(), rtol=1e-11, atol=1e-12)
    # L = 1: y = C.(e^{dA} h_prev + delta u B) + D u
    out, hl = orc.ssm_fwd(u[:, :1], delta[:, :1], A, B[:, :1], C[:, :1], D, hp)
    h1 = torch.exp(delta[:, 0].unsqueeze(-1) * A) * hp + (delta[:, 0] * u[:, 0]).unsqueeze(-1) * B[:, 0].unsqueeze(1)
    y1 = (h1 * C[:, 0].unsqueeze(1)).sum(-1) + D * u[:, 0]
    np.testing.assert_allclose(out[:, 0], y1.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(hl, h1.numpy(), rtol=1e-12, atol=1e-12)


def test_fwd_clamp_semantics():
    # the kernels clamp delta*A to [-88, 88] before exp (mamba_cuda.py:65-70)
    u, delta, A, B, C, D, hp = _inputs(1, 6, 4, seed=9)
    Ab = A.clone()
    Ab[0, 0] = 30.0  # delta*A up to 300 with delta ~ 10
    delta = delta * 100.0
    out_c, hl_c = orc.ssm_fwd(u, delta, Ab, B, C, D, hp, clamp=True)
    h = hp.clone()
    for t in range(u.shape[1]):
        e = torch.exp(torch.clamp(delta[:, t].unsqueeze(-1) * Ab, -88.0, 88.0))
        h = e * h + (delta[:, t] * u[:, t]).unsqueeze(-1) * B[:, t].unsqueeze(1)
    np.testing.assert_allclose(hl_c, h.numpy(), rtol=1e-12)
    _, hl_n = orc.ssm_fwd(u, delta, Ab, B, C, D, hp, clamp=False)
    assert not np.allclose(hl_c, hl_n)  # the clamp is live in this case


@pytest.mark.parametrize("shape", [(1, 9, 5, 16), (2, 31, 12, 16), (3, 17, 70, 8)])
@pytest.mark.parametrize("with_h", [False, True])
def test_bwd_matches_autograd(shape, with_h):
    u, delta, A, B, C, D, hp = _inputs(*shape, seed=11 + sum(shape), h_prev=with_h)
    g = torch.Generator().manual_seed(99)
    dout = torch.randn(u.shape, generator=g, dtype=F64)
    dhl = torch.randn(shape[0], shape[2], shape[3], generator=g, dtype=F64) if with_h else None
    leaves = [x.clone().requires_grad_(True) for x in (u, delta, A, B, C, D)]
    hpl = hp.clone().requires_grad_(True) if with_h else None
    out, hl = torch_ref.selective_scan_seq(*leaves, hpl)
    loss = (out * dout).sum() + ((hl * dhl).sum() if with_h else 0.0)
    loss.backward()
    r = orc.ssm_bwd(u, delta, A, B, C, D, dout, hp, dhl)
    for name, leaf in zip(("du", "ddelta", "dA", "dB", "dC", "dD"), leaves):
        np.testing.assert_allclose(r[name], leaf.grad.numpy(), rtol=1e-10, atol=1e-12, err_msg=name)
    if with_h:
        np.testing.assert_allclose(r["dh_prev"], hpl.grad.numpy(), rtol=1e-10, atol=1e-12)


def _magnitude_sums(u, delta, A, B, C, D, hp, dout, dhl):
    """The running-error magnitudes of dA, dΔ and du by brute force: the sequential restatement run
    on magnitudes (|u|, |B|, |C|, |dout|, |h_prev|, |dh_last|; delta > 0 keeps |delta*u*B| =
    delta*|u|*|B|), its state magnitudes H_t kept and its adjoint magnitudes G_t = dL+/dH_t taken from
    torch autograd (retained gradients)."""
    L = u.shape[1]
    h = hp.abs().clone().requires_grad_(True)
    hs, es, prevs = [], [], []
    for t in range(L):
        e = torch.exp(delta[:, t, :, None] * A[None])
        hn = e * h + (delta[:, t] * u[:, t].abs())[..., None] * B[:, t, None, :].abs()
        hn.retain_grad()
        hs.append(hn), es.append(e.detach()), prevs.append(h.detach())
        h = hn
    out = torch.stack([(hs[t] * C[:, t, None, :].abs()).sum(-1) for t in range(L)], 1)
    ((out * dout.abs()).sum() + (h * dhl.abs()).sum()).backward()
    s = [es[t] * prevs[t] * hs[t].grad for t in range(L)]  # G_t dA_t H_{t-1}
    gB = torch.stack([(B[:, t, None, :].abs() * hs[t].grad).sum(-1) for t in range(L)], 1)
    dA = sum(delta[:, t, :, None] * s[t] for t in range(L)).sum(0)
    dd = torch.stack([(A.abs()[None] * s[t]).sum(-1) for t in range(L)], 1) + u.abs() * gB
    du = (D * dout).abs() + delta * gB
    return dA, dd, du


def test_term_magnitudes_match_autograd():
    """dA_abs, ddelta_abs, du_abs against the brute force above, dD_abs = sum_{b,t} |dout*u|; each is
    at least its output's magnitude, above it where terms cancel, and equal to it when nothing can
    cancel (A > 0 and u, B, C, D, dout, h_prev, dh_last >= 0)."""
    bsz, L, dm, n = 2, 13, 5, 8
    u, delta, A, B, C, D, hp = _inputs(bsz, L, dm, n, seed=61)
    g = torch.Generator().manual_seed(62)
    dout = torch.randn(u.shape, generator=g, dtype=F64)
    dhl = torch.randn(hp.shape, generator=g, dtype=F64)
    r = orc.ssm_bwd(u, delta, A, B, C, D, dout, hp, dhl)
    dA, dd, du = _magnitude_sums(u, delta, A, B, C, D, hp, dout, dhl)
    for name, ref in (("dA_abs", dA), ("ddelta_abs", dd), ("du_abs", du)):
        np.testing.assert_allclose(r[name], ref.numpy(), rtol=1e-10, atol=1e-14, err_msg=name)
    np.testing.assert_allclose(r["dD_abs"], (dout * u).abs().sum((0, 1)).numpy(), rtol=1e-12)
    for name in ("dA", "ddelta", "du", "dD"):
        assert (r[name + "_abs"] >= np.abs(r[name]) * (1 - 1e-12)).all(), name
        assert (r[name + "_abs"] > np.abs(r[name]) + 1e-9).any(), name  # these terms have mixed signs
    pos = [x.abs() for x in (u, A, B, C, D, hp, dout, dhl)]
    r = orc.ssm_bwd(pos[0], delta, pos[1], pos[2], pos[3], pos[4], pos[6], pos[5], pos[7])
    for name in ("dA", "ddelta", "du", "dD"):
        np.testing.assert_allclose(r[name + "_abs"], r[name], rtol=1e-12, err_msg=name)


@pytest.mark.parametrize("bias,softplus,gate", [(True, True, True), (False, True, False), (True, False, False),
                                                (False, False, True)])
def test_transforms_match_autograd(bias, softplus, gate):
    """ssm_fwd_xf / ssm_bwd_xf against torch autograd through softplus(delta + bias), the
    sequential restatement and silu(z) gating (torch.nn.functional library routines)."""
    bsz, L, dm, n = 2, 11, 6, 16
    u, delta, A, B, C, D, hp = _inputs(bsz, L, dm, n, seed=41)
    g = torch.Generator().manual_seed(42)
    raw = torch.randn(bsz, L, dm, generator=g, dtype=F64) * 2.0 - 1.0 if softplus else delta
    db = 0.5 * torch.randn(dm, generator=g, dtype=F64) if bias else None
    z = torch.randn(bsz, L, dm, generator=g, dtype=F64) if gate else None
    dout = torch.randn(bsz, L, dm, generator=g, dtype=F64)
    dhl = torch.randn(bsz, dm, n, generator=g, dtype=F64)
    leaves = [x.clone().requires_grad_(True) for x in (u, raw, A, B, C, D, hp)]
    dbl = db.clone().requires_grad_(True) if bias else None
    zl = z.clone().requires_grad_(True) if gate else None
    d = leaves[1] + dbl if bias else leaves[1]
    if softplus:
        d = torch.nn.functional.softplus(d)
    out, hl = torch_ref.selective_scan_seq(leaves[0], d, *leaves[2:6], leaves[6])
    if gate:
        out = out * torch.nn.functional.silu(zl)
    ((out * dout).sum() + (hl * dhl).sum()).backward()
    o, h, _ = orc.ssm_fwd_xf(u, raw, A, B, C, D, hp, db, softplus, z)
    np.testing.assert_allclose(o, out.detach().numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(h, hl.detach().numpy(), rtol=1e-11, atol=1e-12)
    r = orc.ssm_bwd_xf(u, raw, A, B, C, D, dout, hp, dhl, db, softplus, z)
    for name, leaf in zip(("du", "ddelta", "dA", "dB", "dC", "dD", "dh_prev"), leaves):
        np.testing.assert_allclose(r[name], leaf.grad.numpy(), rtol=1e-10, atol=1e-12, err_msg=name)
    if bias:
        np.testing.assert_allclose(r["ddelta_bias"], dbl.grad.numpy(), rtol=1e-10, atol=1e-12)
    if gate:
        np.testing.assert_allclose(r["dz"], zl.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_bwd_finite_differences():
    """Central differences of the oracle's own forward pin its backward."""
    bsz, L, dm, n = 2, 6, 3, 4
    u, delta, A, B, C, D, hp = _inputs(bsz, L, dm, n, seed=21)
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(bsz, L, dm, generator=g, dtype=F64)
    dhl = torch.randn(bsz, dm, n, generator=g, dtype=F64)
    args = [x.numpy().copy() for x in (u, delta, A, B, C, D, hp)]
    names = ["du", "ddelta", "dA", "dB", "dC", "dD", "dh_prev"]
    r = orc.ssm_bwd(*args[:6], dout, args[6], dhl)

    def loss(a):
        o, h = orc.ssm_fwd(*a)
        return float((o * dout.numpy()).sum() + (h * dhl.numpy()).sum())

    eps = 1e-6
    for i, name in enumerate(names):
        num = np.zeros_like(args[i])
        for idx in np.ndindex(args[i].shape):
            ap = [x.copy() for x in args]
            am = [x.copy() for x in args]
            ap[i][idx] += eps
            am[i][idx] -= eps
            num[idx] = (loss(ap) - loss(am)) / (2 * eps)
        np.testing.assert_allclose(r[name], num, rtol=1e-6, atol=1e-7, err_msg=name)


def test_bwd_closed_form_identities():
    u, delta, A, B, C, D, hp = _inputs(2, 50, 11, seed=8)
    dout = torch.randn(u.shape, generator=torch.Generator().manual_seed(1), dtype=F64)
    r = orc.ssm_bwd(u, delta, A, B, C, D, dout, hp, None)
    # dD = sum_{b,t} dout*u
    np.testing.assert_allclose(r["dD"], (dout * u).sum((0, 1)).numpy(), rtol=1e-12)
    # A = 0, delta const: dh_prev = sum_t dout_t C_t (g never decays)
    r0 = orc.ssm_bwd(u, delta, torch.zeros_like(A), B, C, D, dout, hp, None)
    np.testing.assert_allclose(r0["dh_prev"], torch.einsum("bld,bln->bdn", dout, C).numpy(), rtol=1e-11)
    # dC = sum_d dout * h_t for the last step (h_t = h_last)
    out, hl = orc.ssm_fwd(u, delta, A, B, C, D, hp)
    np.testing.assert_allclose(r["dC"][:, -1], torch.einsum("bd,bdn->bn", dout[:, -1], torch.from_numpy(hl)).numpy(),
                               rtol=1e-11)


def test_bwd_deterministic():
    u, delta, A, B, C, D, hp = _inputs(2, 40, 150, seed=4)
    dout = torch.randn(u.shape, generator=torch.Generator().manual_seed(2), dtype=F64)
    r1 = orc.ssm_bwd(u, delta, A, B, C, D, dout, hp, None)
    r2 = orc.ssm_bwd(u, delta, A, B, C, D, dout, hp, None)
    for k in r1:
        assert np.array_equal(r1[k], r2[k]), k


@pytest.mark.parametrize("shape", [(2, 3, 50, 4), (1, 1, 1, 7), (4, 1000, 8)])
def test_pscan_matches_sequential(shape):
    g = torch.Generator().manual_seed(7)
    A = 0.9 + 0.1 * torch.rand(shape, generator=g, dtype=F64)
    X = torch.randn(shape, generator=g, dtype=F64)
    H = orc.pscan_fwd(A, X)
    np.testing.assert_allclose(H, torch_ref.pscan_seq(A, X).numpy(), rtol=1e-12, atol=1e-12)


def test_pscan_special_cases():
    g = torch.Generator().manual_seed(8)
    X = torch.randn(3, 2, 64, 5, generator=g, dtype=F64)
    # A = 1 -> cumsum
    np.testing.assert_allclose(orc.pscan_fwd(torch.ones_like(X), X), torch.cumsum(X, 2).numpy(), rtol=1e-12, atol=1e-12)
    # A = 0 -> X
    np.testing.assert_array_equal(orc.pscan_fwd(torch.zeros_like(X), X), X.numpy())
    # constant a -> H_t = sum_s a^{t-s} X_s
    a = 0.95
    H = orc.pscan_fwd(torch.full_like(X, a), X)
    t = torch.arange(64, dtype=torch.float64)
    W = torch.tril(a ** (t.view(-1, 1) - t.view(1, -1)))
    np.testing.assert_allclose(H, torch.einsum("ts,bdsn->bdtn", W, X).numpy(), rtol=1e-10, atol=1e-12)
    # A_0 has no effect
    A = torch.rand(X.shape, generator=g, dtype=F64)
    A2 = A.clone()
    A2[:, :, 0] = 123.0
    np.testing.assert_array_equal(orc.pscan_fwd(A, X), orc.pscan_fwd(A2, X))


def test_pscan_bwd_matches_autograd():
    g = torch.Generator().manual_seed(10)
    A = (0.5 + 0.5 * torch.rand(2, 3, 37, 4, generator=g, dtype=F64)).requires_grad_(True)
    X = torch.randn(2, 3, 37, 4, generator=g, dtype=F64).requires_grad_(True)
    dH = torch.randn(2, 3, 37, 4, generator=g, dtype=F64)
    H = torch_ref.pscan_seq(A, X)
    (H * dH).sum().backward()
    dA, dX = orc.pscan_bwd(A.detach(), H.detach(), dH)
    np.testing.assert_allclose(dA, A.grad.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(dX, X.grad.numpy(), rtol=1e-11, atol=1e-12)
    assert np.all(dA[:, :, 0] == 0)
