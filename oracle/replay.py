"""Rollout-side steps of the reference's train_impl (oracle; test infrastructure).

Restates, in numpy, the per-minibatch work around the training step
(native/src/pufferlib.cu:1847-2160):

* ``transpose_102`` — transpose_102 (native/src/kernels.cu:179-188) with the
  rewards' clamp to [-1, 1] (clamp_precision_kernel, kernels.cu:197-203).
* ``negamax_advantage`` — k_negamax_adv (native/model/ptcg_model2.cu:287-311):
  per row, t = T-2 .. 0,
      s      = (seat_t == seat_{t+1} ? 1 : -1) * (1 - done_{t+1})
      delta  = min(imp_t, rho_clip) * (r_{t+1} + gamma * v_{t+1} * s - v_t)
      A_t    = delta + gamma * lambda * min(imp_t, c_clip) * s * A_{t+1}
  in float32, the reference's operations in the reference's order;
  A_{T-1} = 0 (the buffer is zeroed first, pufferlib.cu:1966); returns =
  values + advantages (select_copy's copy_values_adv_returns, :1756-1775).
* ``prio_replay`` — prio_replay_cuda (:1455-1591): p_b = (sum_t |A_bt|)^alpha
  (non-finite -> 0), probs = (p + 1e-6) / (sum p + 1e-6), cdf = cumulative
  sum, draws with replacement by inverse CDF (first b with cdf_b >= u), and
  importance weights (total_agents * probs[idx])^-beta.  The uniforms come
  from Philox4x32-10 with counter (offset + k, 0, 1) and key seed (the
  reference: cuRAND Philox(seed, subsequence offset + k)); sums in float64.
* ``index_copy`` — index_copy (:1747-1754): dst row idx[i] <- src row i.
* ``train_segments`` — the minibatch loop of train_impl (:1963-2160) over a
  rollout in the train layout: advantage over the whole rollout -> replay
  draw of minibatch_size / horizon segments -> one minibatch step
  (oracle.step) on the drawn segments' rows with their importance weights
  -> ratio and new values written back into the rollout.

Pins (tests/test_oracle_replay.py): the advantage against textbook GAE
(scipy.signal.lfilter discounted sums) through the two-seat perspective
change, against the telescoping closed form at gamma = lambda = 1, against
one-step TD at lambda = 0 and a hand-expanded three-step V-trace case; the
draws against a brute-force count of CDF entries below u and against the
drawn frequencies of many draws; probabilities and weights against closed
forms at alpha = 0, alpha = 1 and beta = 0.
"""
import numpy as np

from .sampler import philox4x32_10

F32 = np.float32


def transpose_102(src, clamp=False):
    out = np.ascontiguousarray(np.swapaxes(np.asarray(src, F32), 0, 1))
    if clamp:
        out = np.minimum(np.maximum(out, F32(-1)), F32(1))
    return out


def negamax_advantage(values, rewards, dones, importance, seats, gamma, lam, rho_clip, c_clip):
    """All inputs (B, T); seats = the actor-seat column of each step's obs row.
    Returns (advantages, returns), float32 (B, T)."""
    v, r, d, imp, seat = (np.asarray(x, F32) for x in (values, rewards, dones, importance, seats))
    B, T = v.shape
    g, l_, rc, cc_ = F32(gamma), F32(lam), F32(rho_clip), F32(c_clip)
    adv = np.zeros((B, T), F32)
    lastlam = np.zeros(B, F32)
    for t in range(T - 2, -1, -1):
        sign = np.where(seat[:, t] == seat[:, t + 1], F32(1), F32(-1))
        s = sign * (F32(1) - d[:, t + 1])
        rho = np.where(imp[:, t] < rc, imp[:, t], rc)
        cc = np.where(imp[:, t] < cc_, imp[:, t], cc_)
        delta = rho * (r[:, t + 1] + g * v[:, t + 1] * s - v[:, t])
        lastlam = delta + g * l_ * cc * s * lastlam
        adv[:, t] = lastlam
    return adv, v + adv


def prio_probs(adv, alpha):
    """(probs, cdf) for (B, T) advantages, float64 sums, float32 results."""
    a = np.abs(np.asarray(adv, np.float64)).sum(1)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        p = np.power(a, float(alpha))
    p[~np.isfinite(p)] = 0.0
    total = p.sum() + 1e-6
    probs = (p + 1e-6) / total
    return probs.astype(F32), np.cumsum(probs).astype(F32)


def replay_uniforms(seed, offset, n):
    k = np.arange(n, dtype=np.uint64) + np.uint64(offset)
    ctr = np.stack([k & np.uint64(0xFFFFFFFF), k >> np.uint64(32), np.zeros(n, np.uint64),
                    np.ones(n, np.uint64)], -1)
    key = np.broadcast_to(np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], np.uint64), (n, 2))
    x = philox4x32_10(ctr, key)[:, 0]
    return ((x >> np.uint32(9)).astype(F32) * F32(2) + F32(1)) * F32(2.0 ** -24)


def draw(cdf, u):
    """First index with cdf >= u (the last index when none is)."""
    return np.minimum(np.searchsorted(np.asarray(cdf, F32), np.asarray(u, F32), side="left"), len(cdf) - 1)


def prio_replay(adv, alpha, n_samples, total_agents, beta, seed, offset):
    probs, cdf = prio_probs(adv, alpha)
    u = replay_uniforms(seed, offset, n_samples)
    idx = draw(cdf, u).astype(np.int32)
    w = np.power(probs[idx].astype(np.float64) * total_agents, -float(beta)).astype(F32)
    return dict(probs=probs, cdf=cdf, u=u, idx=idx, mb_prio=w, offset=offset + n_samples)


def segment_rows(idx, T):
    return (np.asarray(idx, np.int64)[:, None] * T + np.arange(T)[None, :]).reshape(-1).astype(np.int32)


def index_copy(dst, idx, src, dst_rows=None):
    dst = np.array(dst, copy=True)
    n = dst.shape[0] if dst_rows is None else dst_rows
    for i, r in enumerate(np.asarray(idx)):
        if 0 <= r < n:
            dst[r] = src[i]
    return dst


def train_segments(model, opt, obs, actions, logprobs, rewards, dones, values, T, minibatch, hyp, seed,
                   n_minibatches, epoch=0, total_epochs=1, seat_col=None):
    """train_impl's minibatch loop over a (B*T)-row rollout in the train
    layout (rows b*T + t).  rewards are clamped and the importance ratios
    reset to 1 first, as train_impl does before the loop.  Returns the
    per-minibatch draws, the final rollout values / ratios / advantages."""
    from .step import minibatch_step
    obs = np.asarray(obs, F32)
    BT = obs.shape[0]
    B = BT // T
    seats = obs[:, seat_col].reshape(B, T)
    rew = np.minimum(np.maximum(np.asarray(rewards, F32), F32(-1)), F32(1)).reshape(B, T)
    dn = np.asarray(dones, F32).reshape(B, T)
    vals = np.asarray(values, F32).reshape(B, T).copy()
    ratio = np.ones((B, T), F32)
    mb_segs = minibatch // T
    beta = hyp["prio_beta0"] + (1.0 - hyp["prio_beta0"]) * hyp["prio_alpha"] * epoch / total_epochs
    offset = 0
    draws = []
    for _ in range(n_minibatches):
        adv, ret = negamax_advantage(vals, rew, dn, ratio, seats, hyp["gamma"], hyp["gae_lambda"],
                                     hyp["vtrace_rho_clip"], hyp["vtrace_c_clip"])
        pr = prio_replay(adv, hyp["prio_alpha"], mb_segs, B, beta, seed, offset)
        offset = pr["offset"]
        rows = segment_rows(pr["idx"], T)
        inp = dict(actions=np.asarray(actions, F32)[rows], logprobs=np.asarray(logprobs, F32)[rows],
                   advantages=adv.reshape(-1)[rows], returns=ret.reshape(-1)[rows],
                   values=vals.reshape(-1)[rows], prio=np.repeat(pr["mb_prio"], T))
        res = minibatch_step(model, opt, obs[rows], inp, hyp)
        mb_ratio = res["ratio"].detach().numpy().astype(F32).reshape(mb_segs, T)
        mb_val = res["newvalue"].detach().numpy().astype(F32).reshape(mb_segs, T)
        ratio = index_copy(ratio, pr["idx"], mb_ratio)
        vals = index_copy(vals, pr["idx"], mb_val)
        draws.append(dict(idx=pr["idx"], mb_prio=pr["mb_prio"], probs=pr["probs"], stats=res["stats"]))
    adv, ret = negamax_advantage(vals, rew, dn, ratio, seats, hyp["gamma"], hyp["gae_lambda"],
                                 hyp["vtrace_rho_clip"], hyp["vtrace_c_clip"])
    return dict(draws=draws, values=vals, ratio=ratio, advantages=adv, offset=offset)
