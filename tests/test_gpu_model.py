"""Model / trainer parity on the GPU through the C ABI, against the CPU oracle
on identical seeded inputs and weights.

Tolerances (fp32 path; parity bar: relative 1e-4 on fp32 logits, values and gradients):
* forward output (N, A+1): relative L2 <= 1e-5 and max|d| <= 1e-4 * max(1, max|ref|)
* every parameter-gradient tensor: relative L2 <= 1e-4
* weights after Adam steps: relative L2 <= 1e-4 on the weight blob; the
  update w_after - w_before within relative L2 1e-2 and every element within
  2*lr*steps (Adam's normalised step is a sign function of g near g = 0, so
  elements whose gradient is pure rounding noise may step the other way).
Indices and masks are bit-exact by construction (same fp32 obs rows; the
pointer / id handling is pinned separately in test_gpu_model_ids).
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2, max_rel, d2h, masked_slots_zeroed
from ptcg_amd import dims, params, synth, trainer, native
import oracle.model as om
import oracle.adam as oadam
import oracle.step as ostep
import oracle.ppo as oppo

pytestmark = pytest.mark.gpu

HYP = dict(clip_coef=0.2, vf_clip_coef=0.2, vf_coef=0.5, ent_coef=0.01, max_grad_norm=0.5)


def make(dm, B, seed=0, lr=3e-4):
    ref = om.build(dm, seed=seed)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": ref.to_blob(),
                                 "train": dict(minibatch_size=B, learning_rate=lr, **HYP)})
    return ref, pl


def fwd_check(out_gpu, out_ref):
    scale = max(1.0, float(np.abs(out_ref).max()))
    assert rel_l2(out_gpu, out_ref) < 1e-5, rel_l2(out_gpu, out_ref)
    assert np.abs(out_gpu - out_ref).max() <= 1e-4 * scale


@pytest.mark.parametrize("dm,B,rich", [(dims.tiny(), 16, True), (dims.tiny(heads=1, d=32, ffn=64), 5, True),
                                      (dims.CORE, 8, False), (dims.CORE, 8, True)],
                         ids=["tiny", "tiny_h1", "core", "core_rich"])
def test_forward_matches_oracle(dm, B, rich, cuda):
    ref, pl = make(dm, B, seed=B)
    obs = synth.make_obs(dm, B, seed=B + 1, rich=rich)
    out = trainer.debug_forward(pl, obs)
    fwd_check(out, ref(torch.from_numpy(obs)).detach().numpy())
    pl.close()


def test_debug_forward_rejects_wrong_size(cuda):
    dm = dims.tiny()
    ref, pl = make(dm, 8)
    with pytest.raises(RuntimeError, match="need exactly"):
        trainer.debug_forward(pl, synth.make_obs(dm, 7, seed=0))
    pl.close()


def _grads_check(pl, ref, dm, d_scores, tol=1e-4):
    """Every parameter-gradient tensor within relative L2 `tol` of the
    oracle's.  One exception is measured differently: score_mlp.2.bias is
    sum over rows of d(score), and the softmax-logit gradients of each row sum
    to exactly 0, so the true value is 0 and both sides hold only summation
    rounding; it is bounded by 1e-5 * sum|d(score)| instead."""
    g_gpu = params.blob_to_dict(dm, pl.get_grads())
    g_ref = params.blob_to_dict(dm, ref.grad_blob())
    worst = []
    bound = 1e-5 * float(np.abs(d_scores).sum())
    for name in g_ref:
        r = g_ref[name]
        if name == "score_mlp.2.bias":
            assert abs(float(g_gpu[name][0])) <= bound and abs(float(r[0])) <= bound, (g_gpu[name], r, bound)
            continue
        if not np.any(r):
            assert not np.any(g_gpu[name]), f"{name}: gpu grad nonzero where oracle is exactly 0"
            continue
        worst.append((rel_l2(g_gpu[name], r), name))
    worst.sort(reverse=True)
    assert worst[0][0] < tol, worst[:5]
    return worst


@pytest.mark.parametrize("dm,B,rich", [(dims.tiny(), 16, True), (dims.CORE, 16, False), (dims.CORE, 12, True)],
                         ids=["tiny", "core", "core_rich"])
def test_backward_grads_match_oracle(dm, B, rich, cuda):
    ref, pl = make(dm, B, seed=7)
    obs = synth.make_obs(dm, B, seed=8, rich=rich)
    inp = synth.make_ppo_inputs(dm, obs, seed=9)
    # oracle: forward, PPO loss, autograd backward
    o = torch.from_numpy(obs)
    out = ref(o)
    m0, m1 = dm.offsets()["opt_mask"]
    T = lambda k: torch.from_numpy(inp[k])
    res = oppo.ppo_loss(out.detach(), o[:, m0:m1], T("actions"), T("logprobs"), T("advantages"),
                        T("returns"), T("values"), clip=0.2, vf_clip=0.2, vf_coef=0.5, ent_coef=0.01)
    out.backward(res["grad"])
    # gpu
    d_obs = pl.to_device(obs)
    d_inp = {k: pl.to_device(v) for k, v in inp.items()}
    pl.forward_backward(d_obs, None, d_inp)
    pl.sync()
    dec, pgrad, ratio, nv = pl.buffers()
    fwd_check(d2h(dec, (B, dm.n_opt + 1)), masked_slots_zeroed(out.detach().numpy(), obs[:, m0:m1]))
    assert rel_l2(d2h(pgrad, (B, dm.n_opt + 1)), res["grad"].numpy()) < 1e-4
    assert rel_l2(d2h(ratio, (B,)), res["ratio"].numpy()) < 1e-4
    _grads_check(pl, ref, dm, res["grad"].numpy()[:, :dm.n_opt])
    pl.close()


def test_row_index_path_equals_contiguous(cuda):
    dm = dims.tiny()
    B, R = 8, 40
    ref, pl = make(dm, B, seed=2)
    rows = synth.make_obs(dm, R, seed=3, rich=True)
    inp_all = synth.make_ppo_inputs(dm, rows, seed=4)
    idx = np.random.default_rng(5).choice(R, B, replace=False).astype(np.int32)
    d_rows = pl.to_device(rows)
    d_all = {k: pl.to_device(v) for k, v in inp_all.items()}
    pl.forward_backward(d_rows, pl.to_device(idx, np.int32), d_all)
    pl.sync()
    g_idx = pl.get_grads()
    sel = {k: pl.to_device(v[idx]) for k, v in inp_all.items()}
    pl.forward_backward(pl.to_device(rows[idx]), None, sel)
    pl.sync()
    g_cont = pl.get_grads()
    assert rel_l2(g_idx, g_cont) < 1e-6
    pl.close()


@pytest.mark.parametrize("dm,B,steps", [(dims.tiny(), 16, 3), (dims.CORE, 16, 2)], ids=["tiny", "core"])
def test_adam_steps_match_oracle(dm, B, steps, cuda):
    ref, pl = make(dm, B, seed=11, lr=3e-4)
    w0 = ref.to_blob()
    R = B * 2
    rows = synth.make_obs(dm, R, seed=12)
    inp = synth.make_ppo_inputs(dm, rows, seed=13)
    idx_lists = synth.minibatch_indices(R, B, steps, seed=14)
    opt = oadam.OracleAdam([p for _, p in ref.named_blob_params()], lr=3e-4)
    ostep.run_update(ref, opt, rows, inp, idx_lists, dict(HYP))
    trainer.set_rollout(pl, rows, **inp)
    assert trainer.train(pl, index_lists=idx_lists) == {}      # _C.train returns an empty dict
    lg = trainer.log(pl)
    assert lg["minibatches"] == steps and pl.step_count() == steps
    assert lg["agent_steps"] == R and lg["epoch"] == 1
    assert abs(lg["lr"] - 3e-4) <= 3e-4 * 1e-6      # read back from the device scalar
    assert lg["perf"]["train_forward"] > 0 and lg["perf"]["train"] >= lg["perf"]["train_forward"]
    parts = sum(lg["perf"][k] for k in ("train_model_forward", "train_loss", "train_backward", "train_optimizer"))
    assert abs(parts - lg["perf"]["train_forward"]) <= 1e-6 + 1e-4 * lg["perf"]["train_forward"]
    assert lg["util"]["vram_used_gb"] > 0 and lg["loss"]["kl_skipped"] == lg["loss"]["vf_skipped"] == 0
    assert trainer.log(pl)["loss"] == {}     # the sums were reset by the previous log
    w_gpu, w_ref = pl.get_weights(), ref.to_blob()
    assert rel_l2(w_gpu, w_ref) < 1e-4, rel_l2(w_gpu, w_ref)
    upd_err = rel_l2(w_gpu - w0, w_ref - w0)
    assert upd_err < 1e-2, upd_err
    assert np.abs(w_gpu - w_ref).max() <= 2.0 * 3e-4 * steps
    pl.close()


def test_weights_and_state_round_trip(tmp_path, cuda):
    dm = dims.tiny()
    B = 8
    ref, pl = make(dm, B, seed=21)
    rows = synth.make_obs(dm, B, seed=22)
    inp = synth.make_ppo_inputs(dm, rows, seed=23)
    trainer.set_rollout(pl, rows, **inp)
    trainer.train(pl, index_lists=[np.arange(B, dtype=np.int32)])
    w = pl.get_weights()
    trainer.save_weights(pl, tmp_path / "w.bin")
    assert (tmp_path / "w.bin").stat().st_size == 4 * params.packed_size(dm)
    assert np.array_equal(np.fromfile(tmp_path / "w.bin", np.float32), w)
    trainer.save_state(pl, tmp_path / "s.bin")
    m, v = pl.get_moments()
    _, pl2 = make(dm, B, seed=99)
    trainer.load_state(pl2, tmp_path / "s.bin")
    assert np.array_equal(pl2.get_weights(), w) and pl2.step_count() == 1
    m2, v2 = pl2.get_moments()
    assert np.array_equal(m, m2) and np.array_equal(v, v2)
    # continuing from the restored state matches continuing the original
    trainer.set_rollout(pl2, rows, **inp)
    trainer.train(pl, index_lists=[np.arange(B, dtype=np.int32)])
    trainer.train(pl2, index_lists=[np.arange(B, dtype=np.int32)])
    # bit for bit: fixed-order reductions, order-independent table scatters
    assert np.array_equal(pl.get_weights(), pl2.get_weights())
    _, pl3 = make(dm, B, seed=5)
    trainer.load_weights(pl3, tmp_path / "w.bin")
    assert np.array_equal(pl3.get_weights(), w)
    (tmp_path / "bad.bin").write_bytes(b"\0" * 12)
    with pytest.raises(RuntimeError, match="size mismatch"):
        trainer.load_weights(pl3, tmp_path / "bad.bin")
    with pytest.raises(RuntimeError, match="PTCGADM1"):
        trainer.load_state(pl3, tmp_path / "w.bin")
    for p in (pl, pl2, pl3):
        p.close()


def test_gate_vetoes_step(cuda):
    dm = dims.tiny()
    B = 8
    ref, pl = make(dm, B, seed=31)
    rows = synth.make_obs(dm, B, seed=32)
    inp = synth.make_ppo_inputs(dm, rows, seed=33)
    w0 = pl.get_weights()
    # synthetic old log-probs are far from the policy's -> approx KL >> 1e-6
    pl.set_hypers(kl_skip_threshold=1e-6)
    trainer.set_rollout(pl, rows, **inp)
    trainer.train(pl, index_lists=[np.arange(B, dtype=np.int32)])
    lg = trainer.log(pl)
    # a KL veto: kl_skipped counts it, vf_skipped does not (pufferlib.cu:1300-1301)
    assert lg["loss"]["kl_skipped"] == 1 and lg["loss"]["vf_skipped"] == 0 and pl.step_count() == 0
    assert lg["gate"] == 0.0
    assert np.array_equal(pl.get_weights().view(np.uint32), w0.view(np.uint32))
    m, v = pl.get_moments()
    assert not m.any() and not v.any()
    # a value-loss veto (KL test off): both counters count it; the counters
    # were reset by the log above, the gate keeps its last value until a step
    pl.set_hypers(kl_skip_threshold=0.0, vf_skip_threshold=1e-9)
    trainer.train(pl, index_lists=[np.arange(B, dtype=np.int32)] * 2)
    lg = trainer.log(pl)
    assert lg["loss"]["kl_skipped"] == 2 and lg["loss"]["vf_skipped"] == 2 and pl.step_count() == 0
    # both tests pass: the step applies and no counter moves
    pl.set_hypers(kl_skip_threshold=1e9, vf_skip_threshold=1e9)
    trainer.train(pl, index_lists=[np.arange(B, dtype=np.int32)])
    lg = trainer.log(pl)
    assert lg["loss"]["kl_skipped"] == 0 and lg["loss"]["vf_skipped"] == 0 and pl.step_count() == 1
    assert lg["gate"] == 1.0
    pl.close()


def test_pointers_into_padding_and_no_valid_tokens(cuda):
    """Option pointers that select padded tokens (whose trunk rows are then
    computed although they are no keys) and a sample with no valid token at
    all: the compact trunk layout must give the full-length results."""
    dm = dims.tiny()
    B = 8
    ref, pl = make(dm, B, seed=51)
    obs = synth.make_obs(dm, B, seed=52, rich=True, max_pad=dm.l_tok // 2)
    off = dm.offsets()
    ti = obs[:, off["tok_int"][0]:off["tok_int"][1]].reshape(B, dm.l_tok, dm.tok_int)
    oi = obs[:, off["opt_int"][0]:off["opt_int"][1]].reshape(B, dm.n_opt, dm.opt_int)
    tf = obs[:, off["tok_float"][0]:off["tok_float"][1]].reshape(B, dm.l_tok, dm.tok_f)
    rng = np.random.default_rng(53)
    for i in range(B):
        pad = np.flatnonzero(ti[i, :, 1] <= 0)
        if pad.size:
            ti[i, pad, 0] = rng.integers(0, dm.n_cards, pad.size)      # padded tokens carry content
            tf[i, pad] = rng.standard_normal((pad.size, dm.tok_f))
            oi[i, 0, 1] = pad[0] + 1
            oi[i, 1, 2] = pad[-1] + 1
    ti[3, :, 1] = 0                                                     # sample 3: every token padded
    inp = synth.make_ppo_inputs(dm, obs, seed=54)
    o = torch.from_numpy(obs)
    out = ref(o)
    m0, m1 = off["opt_mask"]
    T = lambda k: torch.from_numpy(inp[k])
    res = oppo.ppo_loss(out.detach(), o[:, m0:m1], T("actions"), T("logprobs"), T("advantages"),
                        T("returns"), T("values"), clip=0.2, vf_clip=0.2, vf_coef=0.5, ent_coef=0.01)
    out.backward(res["grad"])
    pl.forward_backward(pl.to_device(obs), None, {k: pl.to_device(v) for k, v in inp.items()})
    pl.sync()
    dec, _, _, _ = pl.buffers()
    fwd_check(d2h(dec, (B, dm.n_opt + 1)), masked_slots_zeroed(out.detach().numpy(), obs[:, m0:m1]))
    _grads_check(pl, ref, dm, res["grad"].numpy()[:, :dm.n_opt])
    pl.close()
