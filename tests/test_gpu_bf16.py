"""Mixed precision (bf16 GEMM and attention products, fp32 LayerNorm,
softmax, loss and accumulation) against the
fp32 oracle.

Tolerances (written here, per the config's proposal): on legal options the
logits |d| <= 2e-2 * max(1, |ref|); value relative error <= 2e-2 (L2 over the
batch); mean masked-softmax KL(ref || bf16) <= 1e-3.  Gradients: every
tensor relative L2 <= 5e-2 and cosine >= 0.998 against the fp32 oracle's
(bf16 rounds each product operand to 8 bits of mantissa, ~4e-3 relative per
element).  Weights after 3 Adam steps: relative L2 <= 1e-3.
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2, d2h
from ptcg_amd import dims, params, synth, trainer
import oracle.model as om
import oracle.adam as oadam
import oracle.step as ostep
import oracle.ppo as oppo

pytestmark = pytest.mark.gpu

HYP = dict(clip_coef=0.2, vf_clip_coef=0.2, vf_coef=0.5, ent_coef=0.01, max_grad_norm=0.5)


def make(dm, B, seed, lr=3e-4):
    st = synth.make_static(dm, seed + 1000) if dm.tables == 1 else None
    ref = om.build(dm, seed=seed, static=st)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": ref.to_blob(), "static": st, "precision": "bf16",
                                 "train": dict(minibatch_size=B, learning_rate=lr, **HYP)})
    return ref, pl


def forward_check(out, want, mask):
    A = mask.shape[1]
    legal = mask != 0
    scale = np.maximum(1.0, np.abs(want[:, :A]))
    assert np.all(np.abs(out[:, :A] - want[:, :A])[legal] <= 2e-2 * scale[legal])
    assert rel_l2(out[:, A], want[:, A]) <= 2e-2
    lw = np.where(legal, want[:, :A], -1e4).astype(np.float64)
    lo = np.where(legal, out[:, :A], -1e4).astype(np.float64)
    lp = lw - np.log(np.exp(lw - lw.max(1, keepdims=True)).sum(1, keepdims=True)) - lw.max(1, keepdims=True)
    lq = lo - np.log(np.exp(lo - lo.max(1, keepdims=True)).sum(1, keepdims=True)) - lo.max(1, keepdims=True)
    kl = (np.exp(lp) * (lp - lq)).sum(1).mean()
    assert kl <= 1e-3, kl


@pytest.mark.parametrize("dm,B", [(dims.CORE, 512), (dims.tiny_frozen(), 16)], ids=["core_b512", "tiny_frozen"])
def test_bf16_forward_within_tolerance(dm, B, cuda):
    ref, pl = make(dm, B, seed=31)
    obs = synth.make_obs(dm, B, seed=32, rich=dm.tables == 1)
    out = trainer.debug_forward(pl, obs)
    with torch.no_grad():
        want = ref(torch.from_numpy(obs)).numpy()
    m0, m1 = dm.offsets()["opt_mask"]
    forward_check(out, want, obs[:, m0:m1])
    pl.close()


def test_bf16_gradients_and_steps(cuda):
    dm, B = dims.CORE, 64
    ref, pl = make(dm, B, seed=41)
    obs = synth.make_obs(dm, B, seed=42)
    inp = synth.make_ppo_inputs(dm, obs, seed=43)
    o = torch.from_numpy(obs)
    out = ref(o)
    m0, m1 = dm.offsets()["opt_mask"]
    T = lambda k: torch.from_numpy(inp[k])
    res = oppo.ppo_loss(out.detach(), o[:, m0:m1], T("actions"), T("logprobs"), T("advantages"), T("returns"),
                        T("values"), clip=0.2, vf_clip=0.2, vf_coef=0.5, ent_coef=0.01)
    out.backward(res["grad"])
    pl.forward_backward(pl.to_device(obs), None, {k: pl.to_device(v) for k, v in inp.items()})
    pl.sync()
    g_gpu = params.blob_to_dict(dm, pl.get_grads())
    g_ref = params.blob_to_dict(dm, ref.grad_blob())
    for name, r in g_ref.items():
        if name == "score_mlp.2.bias" or not np.any(r):
            continue
        a = g_gpu[name].ravel().astype(np.float64)
        b = r.ravel().astype(np.float64)
        cos = a @ b / (np.linalg.norm(a) * np.linalg.norm(b))
        assert rel_l2(a, b) <= 5e-2 and cos >= 0.998, (name, rel_l2(a, b), cos)
    pl.close()
    # three clipped Adam steps track the fp32 oracle
    ref, pl = make(dm, B, seed=44)
    rows = synth.make_obs(dm, 2 * B, seed=45)
    inp = synth.make_ppo_inputs(dm, rows, seed=46)
    idx = synth.minibatch_indices(2 * B, B, 3, seed=47)
    opt = oadam.OracleAdam([p for _, p in ref.named_blob_params()], lr=3e-4)
    ostep.run_update(ref, opt, rows, inp, idx, dict(HYP))
    trainer.set_rollout(pl, rows, **inp)
    trainer.train(pl, index_lists=idx)
    assert rel_l2(pl.get_weights(), ref.to_blob()) <= 1e-3
    pl.close()


def test_bf16_rollout_tracks_fp32(cuda):
    """Config 5's bf16 rollout: the same rows and uniforms through bf16 GEMM
    and attention products draw the fp32 rollout's actions except where a
    draw sits within the logits' bf16 error of a CDF boundary; values and the
    log-probabilities of agreeing draws within bf16 tolerance."""
    dm, n = dims.CORE, 512
    blob = om.build(dm, seed=81).to_blob()
    rows = synth.make_obs(dm, n, seed=82)
    res = {}
    for prec in ("fp32", "bf16"):
        pl = trainer.create_pufferl({"dims": dm, "init_weights": blob, "precision": prec,
                                     "train": dict(minibatch_size=64)})
        try:
            d = pl.to_device(rows)
            a, lp, v = pl.rollout_step(d, n, seed=5, step=9)
            torch.cuda.synchronize()
            res[prec] = (a.numpy(), lp.numpy(), v.numpy())
        finally:
            pl.close()
    a0, l0, v0 = res["fp32"]
    a1, l1, v1 = res["bf16"]
    same = a1 == a0
    assert same.mean() >= 0.97, same.mean()
    assert np.abs(l1[same] - l0[same]).max() <= 5e-2
    assert rel_l2(v1, v0) <= 2e-2
    assert not np.array_equal(v1, v0)     # the products really ran in bf16
