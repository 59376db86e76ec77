"""Parity of the reference model variant on the GPU: static-table chain,
oracle critic, blind-value and belief aux heads (dims.tables = 1,
dims.critic = 1), against the CPU oracle on identical seeded inputs.

Tolerances as for the learned-table model (test_gpu_model.py): forward
relative L2 <= 1e-5; every gradient tensor relative L2 <= 1e-4; weights after
Adam steps relative L2 <= 1e-4.  The static-table chain's scatters (pool
backward, CardVec rows shared by tokens / options / oracle tokens) add in
order-independent fixed point, so repeated calls agree bit for bit
(test_gpu_determinism.py).
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2, d2h, masked_slots_zeroed
from ptcg_amd import dims, params, synth, trainer
import oracle.model as om
import oracle.adam as oadam
import oracle.step as ostep
import oracle.ppo as oppo

pytestmark = pytest.mark.gpu

HYP = dict(clip_coef=0.2, vf_clip_coef=0.2, vf_coef=0.5, ent_coef=0.01, max_grad_norm=0.5)


def make(dm, B, seed=0, lr=3e-4):
    st = synth.make_static(dm, seed + 1000)
    ref = om.build(dm, seed=seed, static=st)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": ref.to_blob(), "static": st,
                                 "train": dict(minibatch_size=B, learning_rate=lr, **HYP)})
    return ref, pl


def test_variant_shapes_and_blob():
    dm = dims.FROZEN
    assert params.packed_size(dm) == 4465812 and len(params.param_order(dm)) == 120
    assert dm.obs_size == 10944


@pytest.mark.parametrize("dm,B", [(dims.tiny_frozen(), 8), (dims.FROZEN, 4), (dims.FROZEN_D128, 4)],
                         ids=["tiny", "frozen", "frozen_d128"])
def test_variant_forward_matches_oracle(dm, B, cuda):
    ref, pl = make(dm, B, seed=3)
    obs = synth.make_obs(dm, B, seed=4, rich=True)
    out = trainer.debug_forward(pl, obs)
    want = ref(torch.from_numpy(obs)).detach().numpy()
    scale = max(1.0, float(np.abs(want).max()))
    assert rel_l2(out, want) < 1e-5, rel_l2(out, want)
    assert np.abs(out - want).max() <= 1e-4 * scale
    pl.close()


def test_static_tables_required(cuda):
    dm = dims.tiny_frozen()
    st = synth.make_static(dm, 1)
    ref = om.build(dm, seed=0, static=st)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": ref.to_blob(), "train": dict(minibatch_size=4)})
    with pytest.raises(RuntimeError, match="static tables not uploaded"):
        trainer.debug_forward(pl, synth.make_obs(dm, 4, seed=0))
    bad = dict(st, card_attacks=np.full_like(st["card_attacks"], dm.n_attacks))
    with pytest.raises(RuntimeError, match="card_attacks"):
        pl.set_static(bad)
    pl.close()


def _oracle_fwd_bwd(ref, dm, obs, inp):
    o = torch.from_numpy(obs)
    out, parts = ref(o, return_parts=True)
    m0, m1 = dm.offsets()["opt_mask"]
    T = lambda k: torch.from_numpy(inp[k])
    res = oppo.ppo_loss(out.detach(), o[:, m0:m1], T("actions"), T("logprobs"), T("advantages"),
                        T("returns"), T("values"), clip=0.2, vf_clip=0.2, vf_coef=0.5, ent_coef=0.01)
    obj = (out * res["grad"]).sum() + ref.aux_loss(o, parts, inp["returns"])
    obj.backward()
    return out.detach().numpy(), res


# frozen_d128: the reference's d128 / h4 / FFN 256 trunk (ptcg_model.cu:19), whose
# d = 128 blocks take the unfused residual / LayerNorm launches (the fused
# kernels own d = 256 rows)
@pytest.mark.parametrize("dm,B", [(dims.tiny_frozen(), 12), (dims.FROZEN, 6), (dims.FROZEN_D128, 6)],
                         ids=["tiny", "frozen", "frozen_d128"])
def test_variant_backward_grads_match_oracle(dm, B, cuda):
    ref, pl = make(dm, B, seed=5)
    obs = synth.make_obs(dm, B, seed=6, rich=True)
    inp = synth.make_ppo_inputs(dm, obs, seed=7)
    out, res = _oracle_fwd_bwd(ref, dm, obs, inp)
    pl.forward_backward(pl.to_device(obs), None, {k: pl.to_device(v) for k, v in inp.items()})
    pl.sync()
    dec, pgrad, _, _ = pl.buffers()
    m0, m1 = dm.offsets()["opt_mask"]
    assert rel_l2(d2h(dec, (B, dm.n_opt + 1)), masked_slots_zeroed(out, obs[:, m0:m1])) < 1e-5
    assert rel_l2(d2h(pgrad, (B, dm.n_opt + 1)), res["grad"].numpy()) < 1e-4
    g_gpu = params.blob_to_dict(dm, pl.get_grads())
    g_ref = params.blob_to_dict(dm, ref.grad_blob())
    bound = 1e-5 * float(np.abs(res["grad"].numpy()[:, :dm.n_opt]).sum())
    worst = []
    for name, r in g_ref.items():
        if name == "score_mlp.2.bias":   # exact value 0 (softmax-logit grads sum to 0 per row)
            assert abs(float(g_gpu[name][0])) <= bound
            continue
        if not np.any(r):
            assert not np.any(g_gpu[name]), name
            continue
        worst.append((rel_l2(g_gpu[name], r), name))
    worst.sort(reverse=True)
    assert worst[0][0] < 1e-4, worst[:5]
    # every stage of the variant received gradient
    for name in ("card_id_emb.weight", "attack_id_emb.weight", "skill_id_emb.weight", "card_mlp.0.weight",
                 "oracle_proj.weight", "critic_readout", "critic_blocks.0.qkv.weight", "aux_hand.weight",
                 "aux_prize.weight", "value_mlp.0.weight", "oracle_value_mlp.2.bias"):
        assert np.any(g_gpu[name]), name
    pl.close()


def test_variant_row_index_path(cuda):
    """Rows and returns read through row_idx equal the gathered minibatch."""
    dm = dims.tiny_frozen()
    B, R = 8, 30
    ref, pl = make(dm, B, seed=8)
    rows = synth.make_obs(dm, R, seed=9, rich=True)
    inp = synth.make_ppo_inputs(dm, rows, seed=10)
    idx = np.random.default_rng(11).choice(R, B, replace=False).astype(np.int32)
    pl.forward_backward(pl.to_device(rows), pl.to_device(idx, np.int32), {k: pl.to_device(v) for k, v in inp.items()})
    pl.sync()
    g_idx = pl.get_grads()
    pl.forward_backward(pl.to_device(rows[idx]), None, {k: pl.to_device(v[idx]) for k, v in inp.items()})
    pl.sync()
    assert rel_l2(g_idx, pl.get_grads()) < 1e-6
    pl.close()


def test_variant_adam_steps_match_oracle(cuda):
    dm, B, steps = dims.tiny_frozen(), 8, 3
    ref, pl = make(dm, B, seed=12)
    w0 = ref.to_blob()
    rows = synth.make_obs(dm, 2 * B, seed=13, rich=True)
    inp = synth.make_ppo_inputs(dm, rows, seed=14)
    idx = synth.minibatch_indices(2 * B, B, steps, seed=15)
    opt = oadam.OracleAdam([p for _, p in ref.named_blob_params()], lr=3e-4)
    ostep.run_update(ref, opt, rows, inp, idx, dict(HYP))
    trainer.set_rollout(pl, rows, **inp)
    trainer.train(pl, index_lists=idx)
    w_gpu, w_ref = pl.get_weights(), ref.to_blob()
    assert rel_l2(w_gpu, w_ref) < 1e-4
    assert rel_l2(w_gpu - w0, w_ref - w0) < 1e-2
    assert np.abs(w_gpu - w_ref).max() <= 2.0 * 3e-4 * steps
    pl.close()
