"""The benchmark configurations at their own sizes, against the oracle.

* config 2 (fp32 forward + backward + PPO loss at B = 512): forward output
  relative L2 <= 1e-5, PPO gradient <= 1e-5, every parameter-gradient
  tensor relative L2 <= 1e-4 (the fp32 parity bar) against the float64 oracle.
* config 4 (bf16 GEMM and attention products): forward at B = 2048 within the
  stated bf16 tolerance (legal logits |d| <= 2e-2 max(1, |ref|), value
  relative L2 <= 2e-2, mean masked-softmax KL <= 1e-3); gradients at B = 512:
  every tensor relative L2 <= 5e-2 and cosine >= 0.998 against the fp32-exact
  oracle.
Config 3 (the 32-step update) is test_gpu_update.py; config 5 (8 192-row
rollout with Gumbel-max draws) is test_gpu_gumbel.py.
"""
import os

import numpy as np
import pytest
import torch

from conftest import rel_l2, d2h, masked_slots_zeroed
from ptcg_amd import dims, params, synth, trainer
import oracle.model as om
import oracle.ppo as oppo

pytestmark = pytest.mark.gpu

HYP = dict(clip_coef=0.2, vf_clip_coef=0.2, vf_coef=0.5, ent_coef=0.01, max_grad_norm=0.5)


def _oracle_fwd_bwd(ref, dm, obs, inp):
    o = torch.from_numpy(obs).double()
    out = ref(o)
    m0, m1 = dm.offsets()["opt_mask"]
    T = lambda k: torch.from_numpy(inp[k]).double()
    res = oppo.ppo_loss(out.detach(), o[:, m0:m1], T("actions"), T("logprobs"), T("advantages"),
                        T("returns"), T("values"), clip=0.2, vf_clip=0.2, vf_coef=0.5, ent_coef=0.01)
    out.backward(res["grad"])
    return out.detach().numpy(), res


def _gpu_fwd_bwd(dm, blob, obs, inp, B, precision):
    pl = trainer.create_pufferl({"dims": dm, "init_weights": blob, "precision": precision,
                                 "train": dict(minibatch_size=B, **HYP)})
    try:
        pl.forward_backward(pl.to_device(obs), None, {k: pl.to_device(v) for k, v in inp.items()})
        pl.sync()
        dec, pgrad, _, _ = pl.buffers()
        return (d2h(dec, (B, dm.n_opt + 1)), d2h(pgrad, (B, dm.n_opt + 1)),
                params.blob_to_dict(dm, pl.get_grads()))
    finally:
        pl.close()


@pytest.mark.timeout(600)
def test_config2_b512_every_gradient(cuda):
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    dm, B = dims.CORE, 512
    ref = om.build(dm, seed=201)
    blob = ref.to_blob()
    ref = om.build(dm, blob=blob, dtype=torch.float64)
    obs = synth.make_obs(dm, B, seed=202)
    inp = synth.make_ppo_inputs(dm, obs, seed=203)
    print("config 2: B=512 fp32 forward+backward vs the float64 oracle", flush=True)
    dec, pgrad, g_gpu = _gpu_fwd_bwd(dm, blob, obs, inp, B, "fp32")
    out, res = _oracle_fwd_bwd(ref, dm, obs, inp)
    m0, m1 = dm.offsets()["opt_mask"]
    want = masked_slots_zeroed(out, obs[:, m0:m1])
    assert rel_l2(dec, want) <= 1e-5, rel_l2(dec, want)
    assert np.abs(dec - want).max() <= 1e-4 * max(1.0, float(np.abs(want).max()))
    assert rel_l2(pgrad, res["grad"].numpy()) <= 1e-5
    g_ref = params.blob_to_dict(dm, ref.grad_blob())
    d_scores = res["grad"].numpy()[:, :dm.n_opt]
    worst = []
    for name, r in g_ref.items():
        if name == "score_mlp.2.bias":   # exact value 0: softmax-logit gradients sum to 0 per row
            assert abs(float(g_gpu[name][0])) <= 1e-5 * float(np.abs(d_scores).sum())
            continue
        assert np.any(r), name
        worst.append((rel_l2(g_gpu[name], r), name))
    worst.sort(reverse=True)
    print("worst gradient tensors:", worst[:4], flush=True)
    assert worst[0][0] <= 1e-4, worst[:5]


def _bf16_forward_check(out, want, mask):
    A = mask.shape[1]
    legal = mask != 0
    scale = np.maximum(1.0, np.abs(want[:, :A]))
    assert np.all(np.abs(out[:, :A] - want[:, :A])[legal] <= 2e-2 * scale[legal])
    assert rel_l2(out[:, A], want[:, A]) <= 2e-2
    lw = np.where(legal, want[:, :A], -1e4).astype(np.float64)
    lo = np.where(legal, out[:, :A], -1e4).astype(np.float64)
    lp = lw - lw.max(1, keepdims=True)
    lp -= np.log(np.exp(lp).sum(1, keepdims=True))
    lq = lo - lo.max(1, keepdims=True)
    lq -= np.log(np.exp(lq).sum(1, keepdims=True))
    kl = (np.exp(lp) * (lp - lq)).sum(1).mean()
    assert kl <= 1e-3, kl
    return kl


@pytest.mark.timeout(600)
def test_config4_bf16_forward_b2048(cuda):
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    dm, B = dims.CORE, 2048
    ref = om.build(dm, seed=211)
    obs = synth.make_obs(dm, B, seed=212)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": ref.to_blob(), "precision": "bf16",
                                 "train": dict(minibatch_size=B, **HYP)})
    try:
        print("config 4: B=2048 bf16 forward vs the oracle", flush=True)
        out = trainer.debug_forward(pl, obs)
    finally:
        pl.close()
    with torch.no_grad():
        want = torch.cat([ref(torch.from_numpy(obs[i:i + 512])) for i in range(0, B, 512)]).numpy()
    m0, m1 = dm.offsets()["opt_mask"]
    kl = _bf16_forward_check(out, want, obs[:, m0:m1])
    print(f"config 4 forward: mean KL {kl:.2e}", flush=True)


@pytest.mark.timeout(600)
def test_config4_bf16_gradients_b512(cuda):
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    dm, B = dims.CORE, 512
    ref = om.build(dm, seed=221)
    blob = ref.to_blob()
    ref = om.build(dm, blob=blob, dtype=torch.float64)
    obs = synth.make_obs(dm, B, seed=222)
    inp = synth.make_ppo_inputs(dm, obs, seed=223)
    print("config 4: B=512 bf16 gradients vs the float64 oracle", flush=True)
    dec, _, g_gpu = _gpu_fwd_bwd(dm, blob, obs, inp, B, "bf16")
    out, res = _oracle_fwd_bwd(ref, dm, obs, inp)
    m0, m1 = dm.offsets()["opt_mask"]
    _bf16_forward_check(dec, masked_slots_zeroed(out, obs[:, m0:m1]), obs[:, m0:m1])
    g_ref = params.blob_to_dict(dm, ref.grad_blob())
    worst = []
    for name, r in g_ref.items():
        if name == "score_mlp.2.bias" or not np.any(r):
            continue
        a = g_gpu[name].ravel().astype(np.float64)
        b = r.ravel().astype(np.float64)
        cos = a @ b / (np.linalg.norm(a) * np.linalg.norm(b))
        worst.append((rel_l2(a, b), cos, name))
    worst.sort(reverse=True)
    print("worst bf16 gradient tensors:", worst[:4], flush=True)
    for e, cos, name in worst:
        assert e <= 5e-2 and cos >= 0.998, (name, e, cos)
