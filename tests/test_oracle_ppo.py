"""Pins of the oracle's PPO loss restatement (CPU).

The hand-written gradient (the native kernel's formulas, pufferlib.cu:1074-1194)
is checked against torch.autograd of the same loss written as an expression,
and the loss against closed-form special cases.
"""
import math

import numpy as np
import pytest
import torch

import oracle.ppo as P

KW = dict(clip=0.2, vf_clip=0.2, vf_coef=0.5, ent_coef=0.01)


def _case(n=64, A=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    out = torch.randn(n, A + 1, generator=g, dtype=torch.float64)
    mask = (torch.rand(n, A, generator=g) < 0.5).double()
    mask[torch.arange(n), torch.randint(0, A, (n,), generator=g)] = 1
    acts = torch.tensor([float(np.random.default_rng(seed + i).choice(np.flatnonzero(mask[i].numpy())))
                         for i in range(n)], dtype=torch.float64)
    old = torch.randn(n, generator=g, dtype=torch.float64) * 0.5 - 2
    adv = torch.randn(n, generator=g, dtype=torch.float64)
    ret = torch.randn(n, generator=g, dtype=torch.float64)
    val = ret - adv + 0.3 * torch.randn(n, generator=g, dtype=torch.float64)
    return out, mask, acts, old, adv, ret, val


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_hand_gradient_equals_autograd(seed):
    out, mask, acts, old, adv, ret, val = _case(seed=seed)
    res = P.ppo_loss(out, mask, acts, old, adv, ret, val, **KW)
    o = out.clone().requires_grad_()
    loss = P.ppo_total_loss(o, mask, acts, old, adv, ret, val, **KW)
    loss.backward()
    assert torch.allclose(res["grad"], o.grad, atol=1e-12, rtol=1e-9)
    assert abs(float(res["stats"][3]) - loss.item()) < 1e-12


def test_clipping_branches_exercised():
    out, mask, acts, old, adv, ret, val = _case(n=256, seed=3)
    res = P.ppo_loss(out, mask, acts, old, adv, ret, val, **KW)
    r = res["ratio"]
    # both the clipped-away (zero pg gradient) and the live branches occur
    assert ((r > 1.2) | (r < 0.8)).any() and ((r < 1.2) & (r > 0.8)).any()


def test_ratio_one_unclipped_policy_gradient():
    out, mask, acts, old, adv, ret, val = _case(n=32, A=8, seed=4)
    logp = torch.log_softmax(P.masked_logits(out[:, :8], mask), 1)
    old = logp.gather(1, acts.long()[:, None]).squeeze(1)     # ratio == 1 exactly
    res = P.ppo_loss(out, mask, acts, old, adv, ret, val, ent_coef=0.0, vf_coef=0.0, clip=0.2, vf_clip=0.2)
    mean, var = P.adv_stats(adv)
    adv_n = (adv - mean) / (var.sqrt() + 1e-8)
    p = logp.exp()
    onehot = torch.zeros_like(p).scatter_(1, acts.long()[:, None], 1.0)
    want = (-adv_n / 32)[:, None] * (onehot - p)          # d(-A r)/dlogits at r = 1
    assert torch.allclose(res["grad"][:, :8], want, atol=1e-12)
    assert torch.allclose(res["ratio"], torch.ones(32, dtype=torch.float64))


def test_equal_advantages_give_no_policy_gradient():
    out, mask, acts, old, adv, ret, val = _case(n=16, A=8, seed=5)
    adv = torch.full_like(adv, 0.7)
    res = P.ppo_loss(out, mask, acts, old, adv, ret, val, ent_coef=0.0, vf_coef=0.5, clip=0.2, vf_clip=0.2)
    assert torch.all(res["grad"][:, :8] == 0)
    assert float(res["stats"][0]) == 0.0


def test_single_legal_option_has_zero_entropy_and_logp():
    n, A = 8, 16
    out, _, _, old, adv, ret, val = _case(n=n, A=A, seed=6)
    mask = torch.zeros(n, A, dtype=torch.float64)
    mask[:, 3] = 1
    acts = torch.full((n,), 3.0, dtype=torch.float64)
    res = P.ppo_loss(out, mask, acts, old, adv, ret, val, **KW)
    assert abs(float(res["stats"][2])) < 1e-12                    # entropy
    assert torch.allclose(res["ratio"], torch.exp(-old))           # logp(action) = 0
    assert torch.all(res["grad"][:, :A] == 0)                      # p = onehot -> no logit grad


def test_masked_options_get_exactly_zero_gradient_and_probabilities_sum_to_one():
    out, mask, acts, old, adv, ret, val = _case(n=64, A=16, seed=7)
    res = P.ppo_loss(out, mask, acts, old, adv, ret, val, **KW)
    assert torch.all(res["grad"][:, :16][mask == 0] == 0)
    logp = torch.log_softmax(P.masked_logits(out[:, :16], mask), 1)
    assert torch.allclose((logp.exp() * mask).sum(1), torch.ones(64, dtype=torch.float64), atol=1e-12)
    ent = -(logp.exp() * logp).sum(1)
    assert torch.all(ent <= torch.log(mask.sum(1)) + 1e-12)
    # softmax logit gradients sum to zero per row (the score-bias identity)
    assert torch.allclose(res["grad"][:, :16].sum(1), torch.zeros(64, dtype=torch.float64), atol=1e-15)


def test_value_clip_branches():
    # v_pred far above v_old + clip with the clipped loss larger -> zero value gradient
    out = torch.zeros(2, 2, dtype=torch.float64)
    out[:, 1] = torch.tensor([1.0, 0.05], dtype=torch.float64)
    mask = torch.ones(2, 1, dtype=torch.float64)
    acts = torch.zeros(2, dtype=torch.float64)
    old = torch.zeros(2, dtype=torch.float64)
    adv = torch.tensor([0.0, 1.0], dtype=torch.float64)
    ret = torch.tensor([2.0, 0.0], dtype=torch.float64)
    val = torch.zeros(2, dtype=torch.float64)
    res = P.ppo_loss(out, mask, acts, old, adv, ret, val, **KW)
    # row 0: v=1, clipped 0.2: (0.2-2)^2 > (1-2)^2 -> clipped branch, |v-v_old| > clip -> 0
    assert res["grad"][0, 1] == 0
    # row 1: v=0.05 inside the clip: both losses equal -> unclipped branch (v - R) / N * vf_coef
    assert abs(float(res["grad"][1, 1]) - 0.5 * 0.05 / 2) < 1e-15


def test_kl_gate_semantics():
    assert P.kl_gate(0.01, 0.1, 0.05, 0.5) == 1.0
    assert P.kl_gate(0.06, 0.1, 0.05, 0.5) == 0.0
    assert P.kl_gate(float("nan"), 0.1, 0.05, 0.5) == 0.0     # fail closed
    assert P.kl_gate(float("nan"), 0.1, 0.0, 0.5) == 1.0      # disabled test
    assert P.kl_gate(0.01, float("inf"), 0.05, 0.5) == 0.0
