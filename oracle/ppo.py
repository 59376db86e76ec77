"""Native PPO clipped loss, forward statistics and hand-written gradient
(oracle; test infrastructure).

Restates ``ppo_var_mean`` (native/src/pufferlib.cu:1307-1363),
``ppo_discrete_head``/``load_logit_masked`` (:949-997) and
``ppo_loss_compute`` (:1010-1248) for one discrete head of ``A`` options,
``T_seq = 1``, no league tag, importance weight ``prio`` per row:

* advantage normalised per minibatch: (adv - mean) / (sqrt(var_unbiased) + 1e-8)
* masked logits: mask == 0 -> -1e4
* ratio = exp(logp(action) - old_logp)
* pg = max(-w*adv_n*ratio, -w*adv_n*clip(ratio, 1-c, 1+c))
* v_loss = 0.5*max((v-R)^2, (v_old + clip(v - v_old, +-vf_clip) - R)^2)
* total = (pg + vf_coef*v_loss - ent_coef*entropy) / N

``ppo_loss`` returns the kernel's gradient formulas (pufferlib.cu:1074-1194);
``ppo_total_loss`` is the same loss written as a differentiable expression so
tests can check those gradients against torch.autograd.
"""
import torch

LOSS_NAMES = ("pg", "vf", "ent", "total", "old_approx_kl", "approx_kl", "clipfrac")


def adv_stats(adv):
    n = adv.numel()
    mean = adv.sum() / n
    var = ((adv - mean) ** 2).sum() / (n - 1)
    return mean, var


def masked_logits(scores, mask):
    return torch.where(mask == 0, torch.full_like(scores, -1e4), scores)


def ppo_loss(out, mask, actions, old_logp, adv, returns, values, *, clip=0.2,
             vf_clip=0.2, vf_coef=0.5, ent_coef=0.01, prio=None):
    """out (N, A+1) = [scores || value]; returns dict with grad (N, A+1),
    the 7 loss statistics (summed over rows, already /N), ratio, newvalue."""
    N, A1 = out.shape
    A = A1 - 1
    scores, vpred = out[:, :A], out[:, A]
    w = torch.ones(N, dtype=out.dtype) if prio is None else prio
    inv = 1.0 / N
    l = masked_logits(scores, mask)
    lse = torch.logsumexp(l, dim=1)
    logp = l - lse[:, None]
    p = torch.exp(logp)
    ent = -(p * logp).sum(1)
    act = actions.long()
    lp_act = logp.gather(1, act[:, None]).squeeze(1)
    logratio = lp_act - old_logp
    ratio = torch.exp(logratio)

    mean, var = adv_stats(adv)
    adv_n = (adv - mean) / (torch.sqrt(var) + 1e-8)
    wa = -w * adv_n
    pg1 = wa * ratio
    pg2 = wa * torch.clamp(ratio, 1 - clip, 1 + clip)
    pg = torch.maximum(pg1, pg2)

    d_ratio = wa * inv
    off = (pg2 > pg1) & ((ratio <= 1 - clip) | (ratio >= 1 + clip))
    d_ratio = torch.where(off, torch.zeros_like(d_ratio), d_ratio)
    dnl = d_ratio * ratio
    d_ent = inv * (-ent_coef)
    onehot = torch.zeros_like(p).scatter_(1, act[:, None], 1.0)
    g_logits = onehot * dnl[:, None] - p * dnl[:, None] \
        + d_ent * p * (-ent[:, None] - logp)

    v_err = vpred - values
    v_clipped = values + torch.clamp(v_err, -vf_clip, vf_clip)
    vl_u = (vpred - returns) ** 2
    vl_c = (v_clipped - returns) ** 2
    v_loss = 0.5 * torch.maximum(vl_u, vl_c)
    use_c = vl_c > vl_u
    inside = (v_err >= -vf_clip) & (v_err <= vf_clip)
    d_v = torch.where(use_c, torch.where(inside, v_clipped - returns,
                                         torch.zeros_like(vpred)),
                      vpred - returns)
    g_value = inv * vf_coef * d_v

    grad = torch.cat([g_logits, g_value[:, None]], dim=1)
    stats = torch.stack([
        (pg * inv).sum(), (v_loss * inv).sum(), (ent * inv).sum(),
        ((pg + vf_coef * v_loss - ent_coef * ent) * inv).sum(),
        (-logratio * inv).sum(), (((ratio - 1) - logratio) * inv).sum(),
        ((torch.abs(ratio - 1) > clip).to(out.dtype) * inv).sum()])
    return dict(grad=grad, stats=stats, ratio=ratio, newvalue=vpred.clone(),
                adv_mean=mean, adv_var=var)


def ppo_total_loss(out, mask, actions, old_logp, adv, returns, values, *,
                   clip=0.2, vf_clip=0.2, vf_coef=0.5, ent_coef=0.01, prio=None):
    """The same total loss as a differentiable expression (autograd check)."""
    N, A1 = out.shape
    A = A1 - 1
    scores, vpred = out[:, :A], out[:, A]
    w = torch.ones(N, dtype=out.dtype) if prio is None else prio
    logp = torch.log_softmax(masked_logits(scores, mask), dim=1)
    ent = -(torch.exp(logp) * logp).sum(1)
    ratio = torch.exp(logp.gather(1, actions.long()[:, None]).squeeze(1) - old_logp)
    mean, var = adv_stats(adv.detach())
    adv_n = (adv - mean) / (torch.sqrt(var) + 1e-8)
    pg = torch.maximum(-w * adv_n * ratio, -w * adv_n * torch.clamp(ratio, 1 - clip, 1 + clip))
    v_clipped = values + torch.clamp(vpred - values, -vf_clip, vf_clip)
    v_loss = 0.5 * torch.maximum((vpred - returns) ** 2, (v_clipped - returns) ** 2)
    return ((pg + vf_coef * v_loss - ent_coef * ent) / N).sum()


def kl_gate(approx_kl, v_loss, kl_threshold, vf_threshold):
    """pufferlib.cu:1292-1302: 1.0 = apply the optimizer step; fails closed
    on non-finite statistics; a threshold <= 0 disables its test."""
    import math
    kl_ok = kl_threshold <= 0 or (math.isfinite(approx_kl) and approx_kl <= kl_threshold)
    vf_ok = vf_threshold <= 0 or (math.isfinite(v_loss) and v_loss <= vf_threshold)
    return 1.0 if (kl_ok and vf_ok) else 0.0
