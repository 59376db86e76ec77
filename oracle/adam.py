"""Global-norm gradient clip + Adam, gated (oracle; test infrastructure).

* clip: coef = min(max_norm / (||g||_2 + 1e-6), 1); g *= coef — the
  formula of ``muon_clip_norm`` (native/src/muon.cu:107-114,216-222), which
  is also torch.nn.utils.clip_grad_norm_'s.
* Adam: torch.optim.Adam(betas, eps, weight_decay=0, amsgrad=False)
  semantics with bias correction; the reference has no Adam (its optimizer
  slot runs Muon, muon.cu:209-297), so torch is the specification.
* gate: when the trainer's gate value is 0 the whole step — moments and
  step count included — is skipped (muon.cu:49-105 LOCAL PATCH semantics).
"""
import torch


def clip_coef(grads, max_norm):
    """clip_grad_norm_'s coefficient min(max_norm / (||g|| + 1e-6), 1), with
    ||g|| accumulated in float64 and rounded to fp32."""
    total = torch.sqrt(sum((g.double() ** 2).sum() for g in grads)).float()
    return torch.clamp(max_norm / (total + 1e-6), max=1.0), total


class OracleAdam:
    """Thin wrapper over torch.optim.Adam on a list of parameters."""

    def __init__(self, params, lr=3e-4, betas=(0.9, 0.999), eps=1e-8):
        self.params = list(params)
        self.opt = torch.optim.Adam(self.params, lr=lr, betas=betas, eps=eps,
                                    weight_decay=0.0, foreach=False)

    def step(self, max_grad_norm, gate=1.0):
        """Clip (norm accumulated in float64: torch's fp32 CPU vector_norm
        drifts ~1e-4 relative at 4M elements) then one Adam step."""
        if gate == 0.0:
            return None
        grads = [p.grad for p in self.params if p.grad is not None]
        coef, norm = clip_coef(grads, max_grad_norm)
        for g in grads:
            g.mul_(coef)
        self.opt.step()
        return norm

    def moments(self):
        m, v = [], []
        for p in self.params:
            st = self.opt.state.get(p, {})
            m.append(st["exp_avg"].reshape(-1) if "exp_avg" in st else torch.zeros(p.numel()))
            v.append(st["exp_avg_sq"].reshape(-1) if "exp_avg_sq" in st else torch.zeros(p.numel()))
        return torch.cat(m).numpy(), torch.cat(v).numpy()


def adam_reference(p, g, m, v, step, lr, b1, b2, eps, coef):
    """Elementwise restatement of one clipped Adam update on flat arrays
    (float64 arithmetic), used to pin the torch wrapper on tiny inputs."""
    import numpy as np
    g = g.astype(np.float64) * coef
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g * g
    bc1 = 1 - b1 ** step
    bc2 = 1 - b2 ** step
    p = p - (lr / bc1) * m / (np.sqrt(v) / np.sqrt(bc2) + eps)
    return p, m, v
