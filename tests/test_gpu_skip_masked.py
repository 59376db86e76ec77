"""Masked-option skipping: the option scorer over legal options only.

The PPO loss maps a masked option's score to the constant logit -1e4, so the
score never reaches the loss and its gradient is exactly zero whenever the
row has a legal option; the trainer therefore runs the option scorer only on
legal options (all options of a row with none legal).  Training steps and
rollout samples must match the full scorer (split-reduction order aside),
including a row whose options are all masked; debug_forward still reports
every slot's score, as the reference's does.
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from ptcg_amd import dims, synth, trainer
import oracle.model as om

pytestmark = pytest.mark.gpu


def _rows(dm, n, seed):
    rows = synth.make_obs(dm, n, seed=seed, rich=dm.l_tok < 32)
    inp = synth.make_ppo_inputs(dm, rows, seed=seed + 1)
    off = dm.offsets()["opt_mask"]
    rows[3, off[0]:off[1]] = 0.0          # a row with no legal option (its action stays as drawn)
    return rows, inp


def _run(dm, B, blob, rows, inp, lists, skip, sync_free=False):
    pl = trainer.create_pufferl({"dims": dm, "init_weights": blob, "skip_masked_options": skip,
                                 "sync_free": sync_free,
                                 "train": dict(minibatch_size=B, learning_rate=1e-3, max_grad_norm=0.5)})
    try:
        # rollout and debug forward on the initial weights, then the update
        fwd = trainer.debug_forward(pl, rows[:B])
        acts, lps, vals = pl.rollout_step(pl.to_device(rows), rows.shape[0], seed=91, step=5)
        trainer.set_rollout(pl, rows, **inp)
        trainer.train(pl, index_lists=lists)
        losses = trainer.log(pl)["loss"]
        w = pl.get_weights()
        return losses, w, fwd, acts.numpy(), lps.numpy(), vals.numpy()
    finally:
        pl.close()


@pytest.mark.parametrize("sync_free", [False, True], ids=["host_count", "sync_free"])
@pytest.mark.parametrize("dm", [dims.tiny(), dims.CORE], ids=["tiny", "core"])
def test_skip_masked_matches_full_scorer(dm, sync_free, cuda):
    B = 32 if dm.l_tok < 32 else 64
    blob = om.build(dm, seed=21).to_blob()
    rows, inp = _rows(dm, 4 * B, seed=22)
    lists = synth.minibatch_indices(4 * B, B, 4, seed=24, epochs=1)
    l0, w0, f0, a0, p0, v0 = _run(dm, B, blob, rows, inp, lists, False, sync_free)
    l1, w1, f1, a1, p1, v1 = _run(dm, B, blob, rows, inp, lists, True, sync_free)
    # Adam's first steps are lr * sign(g): elements whose gradient is rounding
    # noise may step the other way (at most 2 * lr per step).  The two paths
    # run GEMMs of different row counts (so different split-K sums); one
    # flipped element alone is ~5e-5 of the weights' L2 norm here, so the L2
    # bound allows a few and the per-element bound caps each
    assert rel_l2(w1, w0) < 1e-4
    assert np.abs(w1 - w0).max() <= 2 * 1e-3 * len(lists) + 1e-6
    for k in ("policy", "value", "entropy", "total"):
        assert abs(l1[k] - l0[k]) <= 1e-5 * max(1.0, abs(l0[k])), k
    # debug_forward scores every slot in both modes
    assert np.abs(f1 - f0).max() <= 1e-5 * max(1.0, float(np.abs(f0).max()))
    same = a1 == a0
    assert same.mean() >= 0.99
    assert np.abs(p1[same] - p0[same]).max() <= 1e-4
    assert np.abs(v1 - v0).max() <= 1e-4 * max(1.0, float(np.abs(v0).max()))
