"""Sync-free compact mode (row count kept on the device, no host read-back).

The compact trunk layout of blind-critic models normally reads its row count
back to the host once per forward; with ``sync_free`` every launch is sized
for the full N * l_seq rows and stops at the device count, so the step stays
stream-ordered.  The same training steps, debug forward and rollout samples
must come out of both modes (summation orders of split reductions may differ,
hence the fp32 tolerance), and the sync-free forward must match the oracle.
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from ptcg_amd import dims, synth, trainer
import oracle.model as om

pytestmark = pytest.mark.gpu


def _run(dm, B, blob, rows, inp, lists, sync_free):
    pl = trainer.create_pufferl({"dims": dm, "init_weights": blob, "sync_free": sync_free,
                                 "train": dict(minibatch_size=B, learning_rate=1e-3, max_grad_norm=0.5)})
    try:
        fwd0 = trainer.debug_forward(pl, rows[:B])
        trainer.set_rollout(pl, rows, **inp)
        trainer.train(pl, index_lists=lists)
        w = pl.get_weights()
        obs = pl.to_device(rows)
        acts, lps, vals = pl.rollout_step(obs, rows.shape[0], seed=77, step=3)
        torch.cuda.synchronize()
        return fwd0, w, acts.numpy(), lps.numpy(), vals.numpy()
    finally:
        pl.close()


@pytest.mark.parametrize("dm", [dims.tiny(), dims.CORE], ids=["tiny", "core"])
def test_sync_free_matches_default_mode(dm, cuda):
    B = 32 if dm.l_tok < 32 else 64
    blob = om.build(dm, seed=5).to_blob()
    rows = synth.make_obs(dm, 4 * B, seed=6, rich=dm.l_tok < 32)
    inp = synth.make_ppo_inputs(dm, rows, seed=7)
    lists = synth.minibatch_indices(4 * B, B, 4, seed=8, epochs=1)
    f0, w0, a0, l0, v0 = _run(dm, B, blob, rows, inp, lists, False)
    f1, w1, a1, l1, v1 = _run(dm, B, blob, rows, inp, lists, True)
    scale = max(1.0, float(np.abs(f0).max()))
    assert np.abs(f1 - f0).max() <= 1e-5 * scale
    assert rel_l2(w1, w0) < 1e-5
    # the sampler draws from the same uniforms: actions agree unless a draw
    # sits within rounding of a CDF boundary
    assert (a1 == a0).mean() >= 0.99
    same = a1 == a0
    assert np.abs(l1[same] - l0[same]).max() <= 1e-4
    assert np.abs(v1 - v0).max() <= 1e-4 * max(1.0, float(np.abs(v0).max()))


def test_sync_free_forward_matches_oracle(cuda):
    dm, B = dims.tiny(), 32
    ref = om.build(dm, seed=9)
    rows = synth.make_obs(dm, B, seed=10, rich=True)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": ref.to_blob(), "sync_free": True,
                                 "train": dict(minibatch_size=B)})
    try:
        out = trainer.debug_forward(pl, rows)
    finally:
        pl.close()
    want = ref(torch.from_numpy(rows)).detach().numpy()
    assert np.abs(out - want).max() <= 1e-4 * max(1.0, float(np.abs(want).max()))


def _grads(B, blob, rows, inp, sync_free):
    dm = dims.CORE
    pl = trainer.create_pufferl({"dims": dm, "init_weights": blob, "sync_free": sync_free,
                                 "train": dict(minibatch_size=B)})
    try:
        d_obs = pl.to_device(rows)
        d_inp = {k: pl.to_device(v) for k, v in inp.items()}
        pl.forward_backward(d_obs, None, d_inp)
        pl.sync()
        dec = pl.buffers()[0]
        out = torch.empty(B * (dm.n_opt + 1), device="cuda")
        from ptcg_amd.native import check, lib
        check(lib().ptcg_transpose_102(out.data_ptr(), dec, 1, out.numel(), 1, 0, None))
        torch.cuda.synchronize()
        return pl.get_grads(), out.cpu().numpy()
    finally:
        pl.close()


def test_sync_free_matches_default_mode_at_full_batch(cuda):
    """At B = 512 the trunk's 256-wide products have between one and four
    tiles per CU: with host row counts their last wave is balanced (the tail
    tiles split K and reduce through the epilogue); sync-free launches cover
    every tile in one pass.  One forward + backward in each mode: the outputs
    and every gradient agree to fp32 accumulation-order accuracy."""
    dm, B = dims.CORE, 512
    blob = om.build(dm, seed=15).to_blob()
    rows = synth.make_obs(dm, B, seed=16)
    inp = synth.make_ppo_inputs(dm, rows, seed=17)
    g0, o0 = _grads(B, blob, rows, inp, False)
    g1, o1 = _grads(B, blob, rows, inp, True)
    assert np.abs(o1 - o0).max() <= 1e-5 * max(1.0, float(np.abs(o0).max()))
    assert rel_l2(g1, g0) < 1e-5
