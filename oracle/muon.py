"""Muon optimizer step (oracle; test infrastructure).

Restates muon_step (native/src/muon.cu:215-297) for a list of parameters
in blob order:

* clip: coef = min(max_norm / (||g||_2 + 1e-6), 1) over all gradients
  (muon_norm_partials / muon_norm_reduce / muon_clip_norm :3-46, :107-114);
  the norm in float64;
* >= 2-D tensors (R x C): Nesterov momentum m = mu m + g', u = g' + mu m
  (muon_nesterov :49-61); X = u / max(||u||_F, 1e-7); five quintic
  Newton-Schulz iterations with the per-iteration coefficients (a, b, c)
  (ns_coeffs :116-122): A = X X^T, X = a X + (b A + c A A) X for wide
  matrices, A = X^T X, X = a X + X (b A + c A A) for tall ones (R > C)
  (:257-282, in float64 here); w = w (1 - lr wd) - lr sqrt(max(1, R/C)) X;
* 1-D tensors: EMA momentum m = mu m + (1 - mu) g', w = w (1 - lr wd_1d)
  - lr (g' + m) (muon_nesterov_ema :63-86);
* a closed gate (0) changes nothing.

Elementwise arithmetic in float32 in the reference's order; momentum state
float32.  Pins (tests/test_oracle_muon.py): the Newton-Schulz map equals
U p(S) V^T from an SVD (p = the five quintics composed, applied to the
normalised singular values), tall and wide; first-step closed forms of both
momentum rules; the gate; the clip coefficient.
"""
import numpy as np
import torch

NS_COEF = ((4.0848, -6.8946, 2.9270), (3.9505, -6.3029, 2.6377), (3.7418, -5.5913, 2.3037),
           (2.8769, -3.1427, 1.2046), (2.8366, -3.0525, 1.2012))
F32 = torch.float32


def newton_schulz(u, eps=1e-7):
    """u (R, C) -> the orthogonalised update, float64."""
    X = u.double()
    X = X / max(float(torch.linalg.norm(X)), eps)
    tall = X.shape[0] > X.shape[1]
    for a, b, c in NS_COEF:
        if tall:
            A = X.T @ X
            B = b * A + c * (A @ A)
            X = a * X + X @ B
        else:
            A = X @ X.T
            B = b * A + c * (A @ A)
            X = a * X + B @ X
    return X


def quintic_chain(s):
    """The five quintics composed, applied to singular values s."""
    s = np.asarray(s, np.float64)
    for a, b, c in NS_COEF:
        s = a * s + b * s ** 3 + c * s ** 5
    return s


class OracleMuon:
    def __init__(self, params, lr, momentum=0.95, weight_decay=0.0, wd_1d=0.0):
        self.params = list(params)
        self.lr, self.mu, self.wd, self.wd_1d = lr, momentum, weight_decay, wd_1d
        self.mom = [torch.zeros_like(p, dtype=F32) for p in self.params]

    @torch.no_grad()
    def step(self, max_norm, gate=True):
        grads = [p.grad.detach().to(F32) for p in self.params]
        norm = float(torch.sqrt(sum((g.double() ** 2).sum() for g in grads)))
        if not gate:
            return norm
        coef = torch.tensor(min(max_norm / (norm + 1e-6), 1.0), dtype=F32)
        mu = torch.tensor(self.mu, dtype=F32)
        lr = torch.tensor(self.lr, dtype=F32)
        one = torch.tensor(1.0, dtype=F32)
        for p, g, m in zip(self.params, grads, self.mom):
            gc = g * coef
            if p.dim() >= 2:
                m.copy_(mu * m + gc)
                u = gc + mu * m
                R = p.shape[0]
                C = p.numel() // R
                X = newton_schulz(u.reshape(R, C)).to(F32).reshape(p.shape)
                scale = torch.tensor(float(np.sqrt(max(1.0, R / C))), dtype=F32)
                wd = torch.tensor(self.wd, dtype=F32)
                p.data.copy_(p.data.to(F32) * (one - lr * wd) - lr * scale * X)
            else:
                m.copy_(mu * m + (one - mu) * gc)
                u = gc + m
                wd = torch.tensor(self.wd_1d, dtype=F32)
                p.data.copy_(p.data.to(F32) * (one - lr * wd) - lr * one * u)
        return norm
