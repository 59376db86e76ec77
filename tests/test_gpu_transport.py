"""Rollout transport (vecenv.h GPU mode): pinned host observations go up per
buffer, the buffer's captured rollout graph runs on the buffer's stream and
the actions come back to pinned host memory.  Checked bit for bit against
the eager rollout step on the same rows and draw step; rewards / terminals
must land on the device unchanged."""
import numpy as np
import pytest
import torch

from ptcg_amd import dims, synth, trainer
from ptcg_amd import transport as tr
from ptcg_amd.native import check, lib
import oracle.model as om

pytestmark = pytest.mark.gpu


def dev_floats(ptr, n):
    """n floats at device address ptr, copied to the host (a [1, n] -> [n, 1]
    transpose is a plain device copy)."""
    buf = torch.empty(n, dtype=torch.float32, device="cuda")
    check(lib().ptcg_transpose_102(buf.data_ptr(), ptr, 1, n, 1, 0, None))
    torch.cuda.synchronize()
    return buf.cpu().numpy()


def test_transport_round_trip_matches_eager(cuda):
    dm, nbuf, apb = dims.CORE, 2, 96
    blob = om.build(dm, seed=121).to_blob()
    pl = trainer.create_pufferl({"dims": dm, "init_weights": blob, "sync_free": True,
                                 "train": dict(minibatch_size=64)})
    x = tr.RolloutTransport(nbuf * apb, nbuf, dm.obs_size)
    try:
        assert x.agents_per_buffer == apb
        step = torch.tensor([7], dtype=torch.int64, device="cuda")
        for b in range(nbuf):
            x.capture_rollout(pl, b, b, 555, step)
        expect = 7
        for t in range(3):
            for b in range(nbuf):
                # the env's writes for this buffer, then the upload (vecenv.h:355-372)
                rows = synth.make_obs(dm, apb, seed=1000 + 10 * t + b)
                sl = x.slice(b)
                x.observations[sl] = rows
                x.rewards[sl] = np.arange(apb, dtype=np.float32) * (t + 1)
                x.terminals[sl] = (np.arange(apb) % (t + 2) == 0).astype(np.float32)
                x.upload(b)
                x.step(pl, b, b)
                got = x.actions[sl, 0].copy()
                lp = dev_floats(x.device_ptr(tr.LOGPROBS), nbuf * apb)[sl]
                vals = dev_floats(x.device_ptr(tr.VALUES), nbuf * apb)[sl]
                assert np.array_equal(dev_floats(x.device_ptr(tr.REWARDS), nbuf * apb)[sl], x.rewards[sl])
                assert np.array_equal(dev_floats(x.device_ptr(tr.TERMINALS), nbuf * apb)[sl], x.terminals[sl])
                d_rows = pl.to_device(rows)
                a, l, v = pl.rollout_step(d_rows, apb, seed=555, step=expect)
                torch.cuda.synchronize()
                assert np.array_equal(got, a.numpy()), (t, b)
                assert np.array_equal(lp, l.numpy()), (t, b)
                assert np.array_equal(vals, v.numpy()), (t, b)
                expect += 1
                assert int(step.item()) == expect
    finally:
        x.close()
        pl.close()


def test_transport_rejects_bad_shapes(cuda):
    with pytest.raises(Exception, match="do not split"):
        tr.RolloutTransport(100, 3, 64)
    dm = dims.tiny()
    pl = trainer.create_pufferl({"dims": dm, "sync_free": True, "train": dict(minibatch_size=16)})
    x = tr.RolloutTransport(32, 2, dm.obs_size + 4)
    try:
        step = torch.zeros(1, dtype=torch.int64, device="cuda")
        with pytest.raises(Exception, match="observation rows"):
            x.capture_rollout(pl, 0, 0, 1, step)
    finally:
        x.close()
        pl.close()


def test_transport_mask_round_trip(cuda):
    """An env-side action mask (MY_ACTION_MASK bytes per agent) goes up with
    its buffer's observations and lands byte for byte; other buffers' slices
    are untouched."""
    x = tr.RolloutTransport(64, 4, 8, num_atns=1, mask_bytes=24)
    try:
        rng = np.random.default_rng(5)
        x.action_mask[:] = rng.integers(0, 256, size=x.action_mask.shape, dtype=np.uint8)
        x.observations[:] = rng.standard_normal(x.observations.shape).astype(np.float32)
        x.upload(2)
        torch.cuda.synchronize()
        dm = torch.empty(64 * 24, dtype=torch.uint8, device="cuda")
        check(lib().ptcg_transpose_102(dm.data_ptr(), x.device_ptr(tr.MASK), 1, 64 * 24 // 4, 1, 0, None))
        dob = dev_floats(x.device_ptr(tr.OBS), 64 * 8).reshape(64, 8)
        torch.cuda.synchronize()
        got = dm.cpu().numpy().reshape(64, 24)
        sl = x.slice(2)
        assert np.array_equal(got[sl], x.action_mask[sl])
        assert np.array_equal(dob[sl], x.observations[sl])
        others = np.ones(64, bool)
        others[sl] = False
        assert np.all(got[others] == 0) and np.all(dob[others] == 0)
    finally:
        x.close()


def test_transport_buffers_overlap(cuda):
    """Four env buffers, each on its own rollout policy (activations) and
    stream: all four forwards are launched before any is waited on, so they
    may run at once, and each buffer's actions, log-probabilities and values
    equal the eager rollout step's on its rows, bit for bit, at every step."""
    dm, nbuf, apb = dims.CORE, 4, 128
    blob = om.build(dm, seed=131).to_blob()
    pl = trainer.create_pufferl({"dims": dm, "init_weights": blob, "sync_free": True, "sampler": "gumbel",
                                 "train": dict(minibatch_size=64)})
    x = tr.RolloutTransport(nbuf * apb, nbuf, dm.obs_size)
    try:
        steps = [torch.tensor([20 + b], dtype=torch.int64, device="cuda") for b in range(nbuf)]
        for b in range(nbuf):
            x.capture_rollout(pl, b, b, 777, steps[b])
        for t in range(3):
            rows = {}
            for b in range(nbuf):
                rows[b] = synth.make_obs(dm, apb, seed=2000 + 10 * t + b)
                x.observations[x.slice(b)] = rows[b]
                x.upload(b)
            for b in range(nbuf):
                x.launch(pl, b, b)
            for b in range(nbuf):
                x.wait(b)
            lp_all = dev_floats(x.device_ptr(tr.LOGPROBS), nbuf * apb)
            v_all = dev_floats(x.device_ptr(tr.VALUES), nbuf * apb)
            for b in range(nbuf):
                sl = x.slice(b)
                a, l, v = pl.rollout_step(pl.to_device(rows[b]), apb, seed=777, step=20 + b + t, buf=nbuf)
                torch.cuda.synchronize()
                assert np.array_equal(x.actions[sl, 0], a.numpy()), (t, b)
                assert np.array_equal(lp_all[sl], l.numpy()), (t, b)
                assert np.array_equal(v_all[sl], v.numpy()), (t, b)
                assert int(steps[b].item()) == 20 + b + t + 1
    finally:
        x.close()
        pl.close()
