"""Rollout path on the GPU: the action sampler against the oracle sampler
(counter RNG + inverse CDF), and the inference-activation forward against the
training forward.

Bar: uniforms bit-exact (integer Philox arithmetic and exact fp32 scaling);
actions identical except on rows whose uniform lies within 1e-5 of a CDF step
(fp32 exp / log rounding may legitimately pick the neighbour there — counted
and bounded); logprobs within 1e-5 where actions agree; values exact.
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from ptcg_amd import dims, synth, trainer, native
import oracle.model as om
import oracle.sampler as osamp

pytestmark = pytest.mark.gpu


def _run_sampler(dec, mask, seed, step, idx=None):
    n, A1 = dec.shape
    d_dec = torch.from_numpy(dec).cuda()
    d_mask = torch.from_numpy(mask).cuda()
    acts = torch.empty(n, device="cuda")
    lps, vals, us = torch.empty_like(acts), torch.empty_like(acts), torch.empty_like(acts)
    native.check(native.lib().ptcg_sample_actions(d_dec.data_ptr(), n, A1 - 1, d_mask.data_ptr(), mask.shape[1],
                                                  idx, seed, step, acts.data_ptr(), lps.data_ptr(),
                                                  vals.data_ptr(), us.data_ptr(), None))
    torch.cuda.synchronize()
    return acts.cpu().numpy(), lps.cpu().numpy(), vals.cpu().numpy(), us.cpu().numpy()


def _compare(dec, mask, seed, step, got):
    acts, lps, vals, us = got
    r_acts, r_lps, r_vals, r_us = osamp.sample(dec, mask, seed, step)
    assert np.array_equal(us, r_us)
    assert np.array_equal(vals, r_vals)
    diff = acts.astype(np.int64) != r_acts
    if diff.any():
        margin = osamp.boundary_margin(dec, mask, r_us)
        assert np.all(margin[diff] < 1e-5), margin[diff]
    assert diff.sum() <= max(2, len(acts) // 1000)
    same = ~diff
    assert np.abs(lps[same] - r_lps[same]).max() < 1e-5
    return diff.sum()


@pytest.mark.parametrize("seed,step", [(0, 0), (12345, 7), (2 ** 40 + 3, 2 ** 33 + 1)])
def test_sampler_matches_oracle(seed, step, cuda):
    rng = np.random.default_rng(seed % 1000)
    n, A = 4096, 64
    dec = (rng.standard_normal((n, A + 1)) * 2).astype(np.float32)
    mask = (rng.random((n, A)) < 0.4).astype(np.float32)
    mask[np.arange(n), rng.integers(0, A, n)] = 1
    _compare(dec, mask, seed, step, _run_sampler(dec, mask, seed, step))


def test_sampler_special_logits_and_single_legal(cuda):
    rng = np.random.default_rng(3)
    n, A = 256, 16
    dec = rng.standard_normal((n, A + 1)).astype(np.float32)
    dec[0, 2] = np.nan
    dec[1, 5] = np.inf
    dec[2, 7] = -np.inf
    mask = np.ones((n, A), np.float32)
    mask[10:] = 0
    pick = rng.integers(0, A, n - 10)
    mask[np.arange(10, n), pick] = 1
    got = _run_sampler(dec, mask, 5, 9)
    _compare(dec, mask, 5, 9, got)
    assert np.array_equal(got[0][10:].astype(np.int64), pick)
    assert got[0][1] == 5     # +inf logit -> +3.4e38: certain choice
    assert np.abs(got[1][10:]).max() < 1e-6


def test_sampler_distribution(cuda):
    A = 12
    logits = np.linspace(-2, 2, A).astype(np.float32)
    mask = np.ones(A, np.float32)
    mask[[3, 7]] = 0
    n = 50000
    dec = np.tile(np.append(logits, 0.0).astype(np.float32), (n, 1))
    acts = _run_sampler(dec, np.tile(mask, (n, 1)), 99, 1)[0].astype(np.int64)
    l = np.where(mask == 0, -1e4, logits).astype(np.float64)
    p = np.exp(l - l.max())
    p /= p.sum()
    cnt = np.bincount(acts, minlength=A)
    assert cnt[3] == 0 and cnt[7] == 0
    k = p > 1e-9
    chi2 = ((cnt[k] - n * p[k]) ** 2 / (n * p[k])).sum()
    assert chi2 < 29.6   # 9 dof, p = 0.0005


@pytest.mark.parametrize("dm,B", [(dims.tiny(), 24), (dims.tiny_frozen(), 24), (dims.CORE, 64)],
                         ids=["tiny", "tiny_frozen", "core"])
def test_rollout_forward_and_sampling(dm, B, cuda):
    st = synth.make_static(dm, 77) if dm.tables == 1 else None
    ref = om.build(dm, seed=21, static=st)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": ref.to_blob(), "static": st,
                                 "train": dict(minibatch_size=8)})
    rows = synth.make_obs(dm, B, seed=22, rich=True)
    d_rows = pl.to_device(rows)
    acts, lps, vals = pl.rollout_step(d_rows, B, seed=4, step=11)
    torch.cuda.synchronize()
    out = ref(torch.from_numpy(rows)).detach().numpy()
    assert rel_l2(vals.numpy(), out[:, -1]) < 1e-5
    m0, m1 = dm.offsets()["opt_mask"]
    mask = rows[:, m0:m1]
    r_acts, r_lps, _, r_us = osamp.sample(out, mask, 4, 11)
    diff = acts.numpy().astype(np.int64) != r_acts
    if diff.any():   # GPU logits differ from the oracle's at 1e-6: only boundary rows may flip
        assert np.all(osamp.boundary_margin(out, mask, r_us)[diff] < 1e-4)
    assert diff.sum() <= 1
    # row-index path: a permuted gather of the rollout rows
    perm = np.random.default_rng(1).permutation(B).astype(np.int32)
    acts2, _, vals2 = pl.rollout_step(d_rows, B, seed=4, step=11, idx=pl.to_device(perm, np.int32))
    torch.cuda.synchronize()
    assert rel_l2(vals2.numpy(), out[perm, -1]) < 1e-5
    # training still works after a rollout on the same weights
    inp = synth.make_ppo_inputs(dm, rows[:8], seed=23)
    trainer.set_rollout(pl, rows[:8], **inp)
    trainer.train(pl, index_lists=[np.arange(8, dtype=np.int32)])
    assert pl.step_count() == 1
    pl.close()
