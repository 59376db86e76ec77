"""Pins of the oracle's clip + Adam (CPU): torch.optim.Adam through the oracle
wrapper vs an elementwise float64 restatement, the first-step closed form,
the clip coefficient, and the gate."""
import numpy as np
import torch

import oracle.adam as A


def _params(seed, n=(37, 5, 128)):
    g = torch.Generator().manual_seed(seed)
    return [torch.nn.Parameter(torch.randn(k, generator=g)) for k in n]


def test_adam_matches_float64_restatement_over_steps():
    ps = _params(0)
    p0 = [p.detach().numpy().astype(np.float64).copy() for p in ps]
    opt = A.OracleAdam(ps, lr=1e-2, betas=(0.9, 0.999), eps=1e-8)
    m = [np.zeros_like(x) for x in p0]
    v = [np.zeros_like(x) for x in p0]
    ref = [x.copy() for x in p0]
    g = torch.Generator().manual_seed(1)
    for step in range(1, 6):
        grads = [torch.randn(p.shape, generator=g) * 3 for p in ps]
        for p, gr in zip(ps, grads):
            p.grad = gr.clone()
        total = np.sqrt(sum(float((gr.double() ** 2).sum()) for gr in grads))
        coef = min(0.5 / (total + 1e-6), 1.0)
        opt.step(0.5)
        for i, gr in enumerate(grads):
            ref[i], m[i], v[i] = A.adam_reference(ref[i], gr.numpy(), m[i], v[i], step, 1e-2, 0.9, 0.999, 1e-8, coef)
    for p, r in zip(ps, ref):
        assert np.allclose(p.detach().numpy(), r, rtol=1e-5, atol=1e-6)


def test_first_step_closed_form():
    ps = _params(2)
    p0 = [p.detach().clone() for p in ps]
    opt = A.OracleAdam(ps, lr=1e-3)
    for p in ps:
        p.grad = torch.randn(p.shape) * 1e-3
    grads = [p.grad.clone() for p in ps]
    opt.step(1e9)
    for p, q, g in zip(ps, p0, grads):
        want = q - 1e-3 * g / (g.abs() + 1e-8)
        assert torch.allclose(p.detach(), want, atol=1e-9, rtol=1e-5)


def test_clip_coefficient():
    gs = [torch.full((4,), 3.0), torch.full((9,), 4.0)]
    coef, total = A.clip_coef(gs, 1.0)
    assert abs(float(total) - np.sqrt(4 * 9 + 9 * 16)) < 1e-5
    # the coefficient is an fp32 quantity, like the kernel's
    assert abs(float(coef) - 1.0 / (np.sqrt(180.0) + 1e-6)) < 1e-7 * float(coef)
    coef, _ = A.clip_coef(gs, 1e6)
    assert float(coef) == 1.0


def test_gate_zero_is_noop():
    ps = _params(3)
    before = [p.detach().clone() for p in ps]
    opt = A.OracleAdam(ps, lr=1e-1)
    for p in ps:
        p.grad = torch.randn(p.shape)
    assert opt.step(0.5, gate=0.0) is None
    for p, b in zip(ps, before):
        assert torch.equal(p.detach(), b)
    m, v = opt.moments()
    assert not m.any() and not v.any()
