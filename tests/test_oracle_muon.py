"""Pins of the Muon oracle (oracle/muon.py): the Newton-Schulz map against
its SVD closed form, first-step closed forms of both momentum rules, the
gate and the clip coefficient."""
import numpy as np
import pytest
import torch

import oracle.muon as omu


@pytest.mark.parametrize("shape", [(24, 40), (40, 24), (16, 16), (1, 32), (48, 7)])
def test_newton_schulz_is_polynomial_of_singular_values(shape):
    """X = U S V^T -> a X + b X X^T X + c (X X^T)^2 X = U (a S + b S^3 + c S^5) V^T
    per iteration, so the whole map is U p(S / ||X||_F) V^T."""
    g = torch.Generator().manual_seed(shape[0] * 100 + shape[1])
    u = torch.randn(*shape, generator=g, dtype=torch.float64)
    U, S, Vh = torch.linalg.svd(u, full_matrices=False)
    s = (S / torch.linalg.norm(u)).numpy()
    want = U @ torch.diag(torch.from_numpy(omu.quintic_chain(s))) @ Vh
    got = omu.newton_schulz(u)
    assert torch.allclose(got, want, rtol=0, atol=1e-9)


def test_newton_schulz_lands_near_orthogonal():
    # singular values of a well-conditioned matrix end in Muon's band
    g = torch.Generator().manual_seed(3)
    u = torch.randn(64, 128, generator=g, dtype=torch.float64)
    sv = torch.linalg.svdvals(omu.newton_schulz(u))
    assert float(sv.min()) > 0.5 and float(sv.max()) < 1.3


def test_first_step_closed_forms():
    torch.manual_seed(0)
    W = torch.nn.Parameter(torch.randn(12, 20))    # wide, scale 1
    T = torch.nn.Parameter(torch.randn(30, 10))    # tall, scale sqrt(3)
    b = torch.nn.Parameter(torch.randn(20))
    W0, T0, b0 = W.detach().clone(), T.detach().clone(), b.detach().clone()
    for p in (W, T, b):
        p.grad = torch.randn_like(p) * 1e-3         # norm far below max_norm: no clipping
    gW, gT, gb = W.grad.clone(), T.grad.clone(), b.grad.clone()
    lr, mu, wd1 = 0.02, 0.95, 0.1
    opt = omu.OracleMuon([W, T, b], lr=lr, momentum=mu, wd_1d=wd1)
    opt.step(max_norm=10.0)
    # from zero momentum the Nesterov output is (1 + mu) g: Newton-Schulz is scale invariant
    assert torch.allclose(W.detach(), W0 - lr * omu.newton_schulz(gW).float(), atol=1e-6)
    assert torch.allclose(T.detach(), T0 - lr * np.sqrt(3.0) * omu.newton_schulz(gT).float(), atol=1e-6)
    # EMA: m = (1 - mu) g, update g + m = (2 - mu) g
    assert torch.allclose(b.detach(), b0 * (1 - lr * wd1) - lr * (2 - mu) * gb, atol=1e-7)
    assert torch.allclose(opt.mom[2], (1 - mu) * gb, atol=1e-9)
    assert torch.allclose(opt.mom[0], gW, atol=1e-9)


def test_gate_and_clip():
    torch.manual_seed(1)
    p = torch.nn.Parameter(torch.randn(8, 8))
    q = torch.nn.Parameter(torch.randn(8))
    p.grad, q.grad = torch.randn(8, 8) * 10, torch.randn(8) * 10
    p0, q0 = p.detach().clone(), q.detach().clone()
    opt = omu.OracleMuon([p, q], lr=0.1, momentum=0.9)
    norm = opt.step(max_norm=1.0, gate=False)
    assert torch.equal(p.detach(), p0) and torch.equal(q.detach(), q0)
    assert all(float(m.abs().max()) == 0.0 for m in opt.mom)
    want = float(torch.sqrt((p.grad.double() ** 2).sum() + (q.grad.double() ** 2).sum()))
    assert abs(norm - want) < 1e-9 * want
    # clipped: the momentum holds g * max_norm / (||g|| + 1e-6)
    opt.step(max_norm=1.0)
    coef = 1.0 / (want + 1e-6)
    assert torch.allclose(opt.mom[0], p.grad * coef, rtol=1e-6)
