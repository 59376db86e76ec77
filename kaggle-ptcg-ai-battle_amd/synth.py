"""Seeded synthetic observation rows and PPO minibatch inputs.

Rows follow the obs layout of ptcg/rl/buffers.py (via :func:`dims.build_offsets`):
ids are stored as fp32.  Distributions (per row):

* tokens: a valid prefix of ``l_tok - pad`` tokens, ``pad`` uniform in
  [0, max_pad]; valid tokens carry card id U[0, n_cards), zone 1, owner 1,
  tool ids 0 and ``tok_f`` features ~ N(0,1); padded tokens are all zero
  (zone 0 marks padding, ptcg_model.cu:360-367).
* options: each of ``n_opt`` slots legal with p = 0.4, redrawn until at least
  one is legal; a legal slot has type U[1,17), ptr1 = a valid token + 1,
  ptr2 = 0 or a valid token + 1 (p = 1/2 each), card id U[0, n_cards),
  ``opt_f`` features ~ N(0,1); illegal slots are zero; opt_mask = legal.
* global_f ~ N(0,1); dec_int zero; dec_float ~ N(0,1).
* oracle block (models with the oracle critic only, else zero): each of the
  24 opp-hand and 8 my-prize slots holds (id, count/4) and each of the 24
  split slots (id, deck/4, prize/4), id U[1, n_cards) with p = 0.6 else
  empty (0), counts U{1..4}; valid tokens of such models carry zone
  U[1, n_zones) (so MY_UNSEEN = 9 tokens occur) instead of 1.

``rich=True`` additionally exercises the id paths the default leaves at 0
(tool ids, attack ids, decision ids, out-of-range and negative ids that the
model clamps), for parity tests.

PPO inputs: action uniform over the legal set, old log-prob ~ N(-2, 0.5),
advantage ~ N(0,1), return ~ N(0,1), old value = return - advantage
(the reference defines returns = values + advantages, pufferlib.cu:1773).
"""
import numpy as np


def make_obs(dims, n, seed, max_pad=None, rich=False):
    rng = np.random.Generator(np.random.PCG64(seed))
    off = dims.offsets()
    L, T = dims.l_tok, dims.tok_int
    if max_pad is None:
        max_pad = L // 2
    obs = np.zeros((n, dims.obs_size), dtype=np.float32)
    pads = rng.integers(0, max_pad + 1, size=n)
    for i in range(n):
        row = obs[i]
        nv = L - int(pads[i])
        ti = row[off["tok_int"][0]:off["tok_int"][1]].reshape(L, T)
        tf = row[off["tok_float"][0]:off["tok_float"][1]].reshape(L, dims.tok_f)
        ti[:nv, 0] = rng.integers(0, dims.n_cards, size=nv)
        ti[:nv, 1] = rng.integers(1, dims.n_zones, size=nv) if dims.critic == 1 else 1
        ti[:nv, 2] = 1
        tf[:nv] = rng.standard_normal((nv, dims.tok_f))
        if rich:
            ti[:nv, 1] = rng.integers(1, dims.n_zones + 2, size=nv)   # > n_zones-1 clamps
            ti[:nv, 2] = rng.integers(0, dims.n_owners + 1, size=nv)
            tools = rng.integers(-1, dims.n_cards + 3, size=(nv, 2))
            tools[rng.random((nv, 2)) < 0.6] = 0
            ti[:nv, 3:5] = tools
            ti[:nv, 0][rng.random(nv) < 0.05] = dims.n_cards + 7     # clamps to n_cards-1
            ti[:nv, 0][rng.random(nv) < 0.05] = -3                   # clamps to 0
        # options
        no = dims.n_opt
        legal = rng.random(no) < 0.4
        while not legal.any():
            legal = rng.random(no) < 0.4
        oi = row[off["opt_int"][0]:off["opt_int"][1]].reshape(no, dims.opt_int)
        of = row[off["opt_float"][0]:off["opt_float"][1]].reshape(no, dims.opt_f)
        k = int(legal.sum())
        oi[legal, 0] = rng.integers(1, 17, size=k)
        oi[legal, 1] = rng.integers(0, nv, size=k) + 1
        p2 = rng.integers(0, nv, size=k) + 1
        p2[rng.random(k) < 0.5] = 0
        oi[legal, 2] = p2
        oi[legal, 3] = rng.integers(0, dims.n_cards, size=k)
        of[legal] = rng.standard_normal((k, dims.opt_f))
        if rich:
            oi[legal, 4] = rng.integers(0, dims.n_attacks + 2, size=k)
            oi[legal, 0] = rng.integers(0, dims.n_opt_types + 3, size=k)
        row[off["opt_mask"][0]:off["opt_mask"][1]] = legal
        g0, g1 = off["global_f"]
        row[g0:g1] = rng.standard_normal(g1 - g0)
        f0, f1 = off["dec_float"]
        row[f0:f1] = rng.standard_normal(f1 - f0)
        if dims.critic == 1:
            o0, o1 = off["oracle"]
            row[o0:o1] = _oracle_block(rng, dims, rich)
        if rich:
            d0, d1 = off["dec_int"]
            hi = [dims.n_select_types, dims.n_contexts, dims.n_cards, dims.n_cards,
                  dims.n_attacks, dims.n_attacks, dims.n_cards, dims.n_cards]
            row[d0:d1] = [rng.integers(0, h + 2) for h in hi[:d1 - d0]]
    return obs


def _oracle_block(rng, dims, rich):
    """(24 x (id, c/4)) + (24 x (id, d/4, p/4)) + (8 x (id, c/4))"""
    def ids(k):
        v = rng.integers(1, dims.n_cards, size=k)
        v[rng.random(k) < 0.4] = 0
        if rich:   # out-of-range, negative and the unknown id (n_cards - 1)
            r = rng.random(k)
            v[r < 0.05] = dims.n_cards + 2
            v[(r >= 0.05) & (r < 0.1)] = -2
            v[(r >= 0.1) & (r < 0.15)] = dims.n_cards - 1
        return v.astype(np.float32)
    cnt = lambda k: rng.integers(0 if rich else 1, 5, size=k).astype(np.float32) / 4
    hand = np.stack([ids(24), cnt(24)], 1)
    split = np.stack([ids(24), cnt(24), cnt(24)], 1)
    prize = np.stack([ids(8), cnt(8)], 1)
    return np.concatenate([hand.ravel(), split.ravel(), prize.ravel()])


def make_static(dims, seed):
    """Static card / attack / skill features for the static-table model
    (the engine-derived tables of ptcg/rl/cards.py, synthetic here):
    features ~ N(0, 0.5^2); each card lists up to 4 attack ids and 2 skill
    ids (0 = empty slot), occasionally the same id twice."""
    rng = np.random.Generator(np.random.PCG64(seed))
    NC, NA, NS = dims.n_cards, dims.n_attacks, dims.n_skills
    f = lambda *sh: (0.5 * rng.standard_normal(sh)).astype(np.float32)
    att = rng.integers(1, NA, size=(NC, 4))
    att[rng.random((NC, 4)) < 0.4] = 0
    dup = rng.random(NC) < 0.05
    att[dup, 1] = att[dup, 0]
    sk = rng.integers(1, NS, size=(NC, 2))
    sk[rng.random((NC, 2)) < 0.6] = 0
    return dict(card_static=f(NC, 58), att_static=f(NA, 15), card_text=f(NC, 128),
                att_text=f(NA, 64), skill_text=f(NS, 64),
                card_attacks=att.astype(np.int32), card_skills=sk.astype(np.int32))


def make_ppo_inputs(dims, obs, seed):
    """Per-row PPO minibatch inputs for rows ``obs`` (see module doc)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    n = obs.shape[0]
    m0, m1 = dims.offsets()["opt_mask"]
    mask = obs[:, m0:m1] != 0
    actions = np.empty(n, dtype=np.float32)
    for i in range(n):
        legal = np.flatnonzero(mask[i])
        actions[i] = legal[rng.integers(0, legal.size)]
    logprobs = rng.normal(-2.0, 0.5, n).astype(np.float32)
    advantages = rng.standard_normal(n).astype(np.float32)
    returns = rng.standard_normal(n).astype(np.float32)
    values = (returns - advantages).astype(np.float32)
    return dict(actions=actions, logprobs=logprobs, advantages=advantages,
                returns=returns, values=values)


def minibatch_indices(total_rows, minibatch, n_minibatches, seed, epochs=None):
    """Index lists for a multi-epoch PPO update: each epoch draws a fresh
    permutation of the rollout and cuts it into minibatches; returns
    ``n_minibatches`` int32 arrays of ``minibatch`` row indices."""
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    while len(out) < n_minibatches:
        perm = rng.permutation(total_rows).astype(np.int32)
        per_epoch = total_rows // minibatch
        if epochs is not None:
            per_epoch = min(per_epoch, n_minibatches // epochs)
        for j in range(per_epoch):
            out.append(perm[j * minibatch:(j + 1) * minibatch])
            if len(out) == n_minibatches:
                break
    return out
