"""Rollout-side steps on the GPU against the oracle (oracle/replay.py):
train-layout transposes, the negamax V-trace/GAE advantage, prioritized
segment replay, index copies, and train_impl's whole minibatch loop over a
segment rollout (advantage -> replay draw -> step -> ratio / value
write-back) against the oracle's loop.

Tolerances: transposes, copies, draws and row expansions bit-exact; the
advantage within 2e-5 (1 + |A|) (fp32 recurrences of up to 130 steps, with
fused multiply-adds on the GPU); replay probabilities / weights at relative
1e-5 and the CDF within 2e-6 (fp32 block scan vs float64 cumulative sum);
the training loop's weights at relative L2 1e-4 like the other update tests.
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from ptcg_amd import dims, native, synth, trainer
import oracle.model as om
import oracle.adam as oadam
import oracle.replay as orp

pytestmark = pytest.mark.gpu

P = lambda t: t.data_ptr()


def dev(a, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device="cuda", dtype=dt)


@pytest.mark.parametrize("shape", [(64, 2048, 1), (65, 130, 1), (1, 1000, 1), (8, 37, 4736), (3, 5, 64),
                                   (5, 7, 3), (2, 3, 6)])
@pytest.mark.parametrize("clamp", [0, 1])
def test_transpose_102(shape, clamp, cuda):
    A, B, C = shape
    x = np.random.default_rng(A * B + C).uniform(-3, 3, shape).astype(np.float32)
    src, dst = dev(x), torch.empty(B * A * C, device="cuda")
    native.check(native.lib().ptcg_transpose_102(P(dst), P(src), A, B, C, clamp, None))
    torch.cuda.synchronize()
    want = orp.transpose_102(x, clamp=bool(clamp)).reshape(-1)
    assert np.array_equal(dst.cpu().numpy(), want)


def test_fill(cuda):
    x = torch.zeros(1000003, device="cuda")
    native.check(native.lib().ptcg_fill(P(x), x.numel(), 1.0, None))
    torch.cuda.synchronize()
    assert bool((x == 1.0).all())


def _adv_case(B, T, stride, seed):
    rng = np.random.default_rng(seed)
    v = rng.standard_normal((B, T)).astype(np.float32)
    r = rng.uniform(-1, 1, (B, T)).astype(np.float32)
    d = (rng.random((B, T)) < 0.05).astype(np.float32)
    imp = rng.uniform(0.5, 1.5, (B, T)).astype(np.float32)
    seats = rng.integers(0, 2, (B, T)).astype(np.float32)
    obs = rng.standard_normal((B * T, stride)).astype(np.float32)
    col = min(31, stride - 1)
    obs[:, col] = seats.reshape(-1)
    return v, r, d, imp, seats, obs, col


@pytest.mark.parametrize("B,T,stride", [(2048, 64, 67), (16, 64, 4736), (1, 1, 40), (3, 2, 40), (5, 65, 40),
                                        (4, 130, 40), (7, 63, 40)])
def test_negamax_advantage(B, T, stride, cuda):
    v, r, d, imp, seats, obs, col = _adv_case(B, T, stride, B + T)
    g, l, rc, cc = 0.99, 0.95, 1.0, 0.9
    adv, ret = torch.empty(B * T, device="cuda"), torch.empty(B * T, device="cuda")
    # keep every device array referenced until the kernel has run (a freed
    # temporary's block is handed to the next upload of the same size)
    dv, dr, dd, di, do = dev(v), dev(r), dev(d), dev(imp), dev(obs)
    native.check(native.lib().ptcg_negamax_advantage(P(dv), P(dr), P(dd), P(di), P(do), stride, col, P(adv),
                                                     P(ret), g, l, rc, cc, B, T, None))
    torch.cuda.synchronize()
    want, _ = orp.negamax_advantage(v, r, d, imp, seats, g, l, rc, cc)
    a = adv.cpu().numpy().reshape(B, T)
    assert np.all(np.abs(a - want) <= 2e-5 * (1 + np.abs(want)))
    assert np.all(a[:, -1] == 0)
    assert np.array_equal(ret.cpu().numpy().reshape(B, T), v + a)


def _replay(adv, alpha, n, total_agents, beta, seed, offset_dev):
    B, T = adv.shape
    L = native.lib()
    probs, cdf = torch.empty(B, device="cuda"), torch.empty(B, device="cuda")
    idx = torch.empty(n, dtype=torch.int32, device="cuda")
    mbp = torch.empty(n, device="cuda")
    rows = torch.empty(n * T, dtype=torch.int32, device="cuda")
    rprio = torch.full((B * T,), -7.0, device="cuda")
    dadv = dev(adv)
    native.check(L.ptcg_prio_replay(P(dadv), B, T, alpha, n, total_agents, beta, seed, P(offset_dev), P(probs),
                                    P(cdf), P(idx), P(mbp), P(rows), P(rprio), None))
    torch.cuda.synchronize()
    return dict(probs=probs.cpu().numpy(), cdf=cdf.cpu().numpy(), idx=idx.cpu().numpy(), mb_prio=mbp.cpu().numpy(),
                rows=rows.cpu().numpy(), row_prio=rprio.cpu().numpy())


@pytest.mark.parametrize("B,T,n,kind", [(2048, 64, 16, "normal"), (8064, 4, 100, "normal"), (1, 8, 4, "normal"),
                                        (300, 64, 37, "nan_row"), (64, 64, 20, "zeros")])
def test_prio_replay(B, T, n, kind, cuda):
    rng = np.random.default_rng(B + n)
    adv = (rng.standard_normal((B, T)) * rng.uniform(0.1, 3.0, (B, 1))).astype(np.float32)
    if kind == "nan_row":
        adv[5, 7] = np.nan
    if kind == "zeros":
        adv[:] = 0
    alpha, beta, seed = 0.8, 0.35, 12345
    off = torch.tensor([1000], dtype=torch.int64, device="cuda")
    got = _replay(adv, alpha, n, B, beta, seed, off)
    want = orp.prio_replay(adv, alpha, n, B, beta, seed, 1000)
    assert np.allclose(got["probs"], want["probs"], rtol=1e-5, atol=0)
    assert np.all(np.abs(got["cdf"] - want["cdf"]) <= 2e-6)
    # the draw is the inverse CDF of the GPU's own CDF at the oracle's uniforms
    assert np.array_equal(got["idx"], orp.draw(got["cdf"], want["u"]))
    assert np.array_equal(got["idx"], want["idx"])
    assert np.allclose(got["mb_prio"], want["mb_prio"], rtol=1e-5)
    assert np.array_equal(got["rows"], orp.segment_rows(got["idx"], T))
    rp = got["row_prio"].reshape(B, T)
    for k, b in enumerate(got["idx"]):
        assert np.all(rp[b] == got["mb_prio"][k])
    untouched = np.setdiff1d(np.arange(B), got["idx"])
    assert np.all(rp[untouched] == -7.0)
    assert int(off.item()) == 1000 + n
    # the next call continues the counter stream
    got2 = _replay(adv, alpha, n, B, beta, seed, off)
    want2 = orp.prio_replay(adv, alpha, n, B, beta, seed, 1000 + n)
    assert np.array_equal(got2["idx"], want2["idx"])
    assert int(off.item()) == 1000 + 2 * n


def test_prio_replay_rejects_too_many_segments(cuda):
    L = native.lib()
    B = L.ptcg_prio_replay_max_segments() + 1
    z = torch.zeros(B, device="cuda")
    i = torch.zeros(B, dtype=torch.int32, device="cuda")
    off = torch.zeros(1, dtype=torch.int64, device="cuda")
    rc = L.ptcg_prio_replay(P(z), B, 1, 0.8, 1, B, 0.2, 1, P(off), P(z), P(z), P(i), None, None, None, None)
    assert rc != 0 and b"segments" in L.ptcg_last_error()


def test_index_copy(cuda):
    dst = np.zeros((9, 5), np.float32)
    src = np.random.default_rng(3).standard_normal((6, 5)).astype(np.float32)
    idx = np.array([4, 0, 12, -3, 7, 2], np.int32)
    d, di, ds = dev(dst), dev(idx, torch.int32), dev(src)
    native.check(native.lib().ptcg_index_copy(P(d), P(di), P(ds), 6, 5, 9, None))
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy(), orp.index_copy(dst, idx, src))


HYP = dict(clip_coef=0.2, vf_clip_coef=0.2, vf_coef=0.5, ent_coef=0.01, max_grad_norm=0.5,
           gamma=0.99, gae_lambda=0.95, vtrace_rho_clip=1.0, vtrace_c_clip=1.0, prio_alpha=0.8, prio_beta0=0.2)


@pytest.mark.parametrize("layout", ["TB", "BT"])
def test_segment_training_loop_matches_oracle(layout, cuda):
    """train(pl) on a segment rollout: 16 segments x 8 steps, minibatch 32
    (4 segments), 4 minibatches (replay ratio 1), tiny dims."""
    dm, T, S, B, seed = dims.tiny(), 8, 16, 32, 77
    n = S * T
    ref = om.build(dm, seed=31)
    w0 = ref.to_blob()
    obs = synth.make_obs(dm, n, seed=32, rich=True)
    rng = np.random.default_rng(33)
    obs[:, dm.seat_col()] = rng.integers(0, 2, n).astype(np.float32)
    inp = synth.make_ppo_inputs(dm, obs, seed=34)
    rewards = rng.uniform(-1.5, 1.5, n).astype(np.float32)
    dones = (rng.random(n) < 0.1).astype(np.float32)

    pl = trainer.create_pufferl({"dims": dm, "init_weights": w0, "seed": seed,
                                 "train": dict(minibatch_size=B, learning_rate=1e-3, **HYP)})
    try:
        def lay(a):
            a = np.asarray(a, np.float32).reshape(S, T, -1)
            return np.swapaxes(a, 0, 1).copy() if layout == "TB" else a
        trainer.set_segment_rollout(pl, lay(obs), lay(inp["actions"]), lay(inp["logprobs"]), lay(rewards),
                                    lay(dones), lay(inp["values"]), T, layout=layout)
        trainer.train(pl)
        lg = trainer.log(pl)
        w_gpu = pl.get_weights()
        r = pl.rollout
        vals, ratio, off = r["values"].numpy(), r["ratio"].numpy(), int(r["rng_offset"].item())
        last_idx = r["idx"].numpy()[:B // T]
    finally:
        pl.close()

    opt = oadam.OracleAdam([p for _, p in ref.named_blob_params()], lr=1e-3)
    res = orp.train_segments(ref, opt, obs, inp["actions"], inp["logprobs"], rewards, dones, inp["values"], T, B,
                             dict(HYP), seed, n_minibatches=4, seat_col=dm.seat_col())
    assert off == res["offset"] == 4 * (B // T)
    assert np.array_equal(last_idx, res["draws"][-1]["idx"])
    assert lg["minibatches"] == 4 and lg["agent_steps"] == n and lg["epoch"] == 1
    assert lg["perf"]["train_misc"] > 0 and lg["perf"]["train_forward"] > 0
    assert rel_l2(w_gpu, ref.to_blob()) < 1e-4
    assert np.abs(vals - res["values"].reshape(-1)).max() <= 1e-4 * max(1.0, float(np.abs(res["values"]).max()))
    assert np.abs(ratio - res["ratio"].reshape(-1)).max() <= 1e-4
