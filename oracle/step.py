"""One PPO minibatch step and a multi-minibatch update (oracle; test
infrastructure).  Call order of one minibatch, as in ``train_impl``
(native/src/pufferlib.cu:2039-2105): forward -> PPO loss fwd+bwd ->
backward (grads overwritten, ptcg_model4.cu:15-21) -> gate -> clip + optimizer.
"""
import torch

from .ppo import ppo_loss, kl_gate


def minibatch_step(model, opt, obs, inp, hyp):
    obs = torch.as_tensor(obs)
    off = model.off
    m0, m1 = off["opt_mask"]
    mask = obs[:, m0:m1]
    T = lambda k: torch.as_tensor(inp[k])
    out, parts = model(obs, return_parts=True)
    res = ppo_loss(out.detach(), mask, T("actions"), T("logprobs"), T("advantages"),
                   T("returns"), T("values"), clip=hyp["clip_coef"],
                   vf_clip=hyp["vf_clip_coef"], vf_coef=hyp["vf_coef"],
                   ent_coef=hyp["ent_coef"], prio=T("prio") if "prio" in inp else None)
    for p in model.parameters():
        p.grad = None
    # PPO gradient on [scores || value]; with the oracle critic the aux losses
    # the native backward injects (ptcg_model4.cu:26-61) join the objective
    obj = (out * res["grad"].to(out.dtype)).sum()
    if model.dm.critic == 1:
        obj = obj + model.aux_loss(obs, parts, inp["returns"])
    obj.backward()
    gate = kl_gate(float(res["stats"][5]), float(res["stats"][1]),
                   hyp.get("kl_skip_threshold", 0.0), hyp.get("vf_skip_threshold", 0.0))
    norm = opt.step(hyp["max_grad_norm"], gate)
    res["gate"] = gate
    res["grad_norm"] = norm
    res["out"] = out.detach()
    return res


def run_update(model, opt, rollout_obs, rollout_inp, index_lists, hyp):
    """Config-3 style update: one minibatch step per index list."""
    stats = []
    for idx in index_lists:
        inp = {k: v[idx] for k, v in rollout_inp.items()}
        res = minibatch_step(model, opt, rollout_obs[idx], inp, hyp)
        stats.append(res["stats"])
    return torch.stack(stats)
