"""Pins of the rollout-side oracle (oracle/replay.py) against independent
formulations: textbook GAE computed as scipy.signal.lfilter discounted sums,
the two-seat perspective change that turns the negamax recursion into
ordinary GAE, closed forms (telescoping sum, one-step TD, a hand-expanded
V-trace case), brute-force inverse-CDF counts and drawn frequencies."""
import numpy as np
import pytest
from scipy.signal import lfilter

import oracle.replay as orp


def _episode_gae(Rn, V, nt, gamma, lam):
    """Ordinary GAE of one row of T steps: Rn[t] = reward after step t
    (t <= T-2), nt[t] = 1 - done_t; delta_t = Rn[t] + gamma V_{t+1} nt_{t+1}
    - V_t, A_t = delta_t + gamma lam nt_{t+1} A_{t+1}, A_{T-1} = 0.  Computed
    per episode (runs cut where nt == 0) as discounted sums with lfilter."""
    T = V.shape[0]
    delta = Rn + gamma * V[1:] * nt[1:] - V[:-1]
    A = np.zeros(T)
    end = T - 2
    while end >= 0:
        t0 = end
        while t0 - 1 >= 0 and nt[t0] == 1:
            t0 -= 1
        A[t0:end + 1] = lfilter([1.0], [1.0, -gamma * lam], delta[t0:end + 1][::-1])[::-1]
        end = t0 - 1
    return A


def _inputs(B, T, seed, dones_p=0.0, two_seats=False):
    rng = np.random.default_rng(seed)
    v = rng.standard_normal((B, T)).astype(np.float32)
    r = rng.uniform(-1, 1, (B, T)).astype(np.float32)
    d = (rng.random((B, T)) < dones_p).astype(np.float32)
    seats = rng.integers(0, 2, (B, T)).astype(np.float32) if two_seats else np.zeros((B, T), np.float32)
    return v, r, d, seats


def test_single_seat_no_dones_is_textbook_gae():
    B, T, g, l = 6, 64, 0.99, 0.95
    v, r, d, seats = _inputs(B, T, 1)
    A, ret = orp.negamax_advantage(v, r, d, np.ones((B, T), np.float32), seats, g, l, 1.0, 1.0)
    for b in range(B):
        want = _episode_gae(r[b, 1:].astype(np.float64), v[b].astype(np.float64), np.ones(T), g, l)
        assert np.allclose(A[b], want, rtol=1e-4, atol=2e-5)
    assert np.all(A[:, -1] == 0)
    assert np.array_equal(ret, v + A)


@pytest.mark.parametrize("dones_p", [0.0, 0.1])
def test_two_seats_reduce_to_gae_in_seat0_perspective(dones_p):
    """sigma_t = +1 for seat 0, -1 for seat 1: sigma_t * A_t is ordinary GAE
    of V_t = sigma_t v_t and R_{t+1} = sigma_t r_{t+1} (episodes cut at dones)."""
    B, T, g, l = 8, 64, 1.0, 0.95
    v, r, d, seats = _inputs(B, T, 2, dones_p=dones_p, two_seats=True)
    A, _ = orp.negamax_advantage(v, r, d, np.ones((B, T), np.float32), seats, g, l, 1.0, 1.0)
    for b in range(B):
        sig = np.where(seats[b] == 0, 1.0, -1.0)
        Rn = sig[:-1] * r[b, 1:]                   # R_{t+1} seen from the actor at t, in seat-0 terms
        want = sig * _episode_gae(Rn, sig * v[b], 1.0 - d[b].astype(np.float64), g, l)
        assert np.allclose(A[b], want, rtol=1e-4, atol=5e-5), b


def test_gamma_lambda_one_telescopes():
    B, T = 4, 20
    v, r, d, seats = _inputs(B, T, 3)
    A, _ = orp.negamax_advantage(v, r, d, np.ones((B, T), np.float32), seats, 1.0, 1.0, 1.0, 1.0)
    v64, r64 = v.astype(np.float64), r.astype(np.float64)
    for t in range(T - 1):
        want = r64[:, t + 1:].sum(1) + v64[:, -1] - v64[:, t]
        assert np.allclose(A[:, t], want, rtol=1e-5, atol=1e-5)


def test_lambda_zero_is_one_step_vtrace_td():
    B, T, g = 5, 16, 0.9
    v, r, d, seats = _inputs(B, T, 4, dones_p=0.2, two_seats=True)
    imp = np.random.default_rng(5).uniform(0.3, 2.0, (B, T)).astype(np.float32)
    A, _ = orp.negamax_advantage(v, r, d, imp, seats, g, 0.0, 1.0, 1.0)
    s = np.where(seats[:, :-1] == seats[:, 1:], 1.0, -1.0) * (1.0 - d[:, 1:])
    want = np.minimum(imp[:, :-1], 1.0) * (r[:, 1:] + g * v[:, 1:] * s - v[:, :-1])
    assert np.allclose(A[:, :-1], want, rtol=1e-6, atol=1e-6)


def test_three_step_vtrace_by_hand():
    v = np.array([[0.5, -0.25, 1.0]], np.float32)
    r = np.array([[0.0, 0.75, -1.0]], np.float32)
    d = np.zeros((1, 3), np.float32)
    seats = np.array([[0.0, 1.0, 1.0]], np.float32)
    imp = np.array([[0.5, 2.0, 1.0]], np.float32)
    g, l, rho_c, c_c = 0.9, 0.8, 1.0, 0.7
    A, _ = orp.negamax_advantage(v, r, d, imp, seats, g, l, rho_c, c_c)
    # t = 1: same seat (s = 1), rho = min(2, 1) = 1
    d1 = 1.0 * (-1.0 + 0.9 * 1.0 * 1.0 - (-0.25))
    # t = 0: seat changes (s = -1), rho = 0.5, c = min(0.5, 0.7) = 0.5
    d0 = 0.5 * (0.75 + 0.9 * (-0.25) * (-1.0) - 0.5)
    a0 = d0 + 0.9 * 0.8 * 0.5 * (-1.0) * d1
    assert np.allclose(A[0], [a0, d1, 0.0], rtol=1e-6, atol=1e-7)


def test_prio_probs_closed_forms():
    rng = np.random.default_rng(6)
    adv = rng.standard_normal((7, 9)).astype(np.float32)
    S = np.abs(adv.astype(np.float64)).sum(1)
    p1, c1 = orp.prio_probs(adv, 1.0)
    assert np.allclose(p1, (S + 1e-6) / (S.sum() + 1e-6), rtol=1e-6)
    assert np.allclose(c1, np.cumsum((S + 1e-6) / (S.sum() + 1e-6)), rtol=1e-6)
    p0, _ = orp.prio_probs(adv, 0.0)
    assert np.allclose(p0, (1 + 1e-6) / (7 + 1e-6), rtol=1e-6)
    bad = adv.copy()
    bad[2, 3] = np.nan
    pn, _ = orp.prio_probs(bad, 0.8)
    S8 = np.power(np.where(np.arange(7) == 2, 0.0, S), 0.8)
    S8[2] = 0.0
    assert np.allclose(pn, (S8 + 1e-6) / (S8.sum() + 1e-6), rtol=1e-6)


def test_draw_is_brute_force_inverse_cdf():
    rng = np.random.default_rng(7)
    cdf = np.cumsum(rng.random(50)).astype(np.float32)
    cdf /= cdf[-1]
    u = np.concatenate([rng.random(500).astype(np.float32), cdf[[0, 10, 49]], [np.float32(1.0)]])
    got = orp.draw(cdf, u)
    brute = np.array([min(int((cdf < x).sum()), 49) for x in u])
    assert np.array_equal(got, brute)


def test_draw_frequencies_follow_probs():
    probs = np.array([0.1, 0.4, 0.05, 0.3, 0.15])
    adv = np.repeat(probs[:, None], 4, 1).astype(np.float32)   # row sums 4 p
    res = orp.prio_replay(adv, 1.0, 200000, 5, 0.0, seed=123, offset=0)
    freq = np.bincount(res["idx"], minlength=5) / 200000
    sd = np.sqrt(probs * (1 - probs) / 200000)
    assert np.all(np.abs(freq - probs) < 5 * sd)
    assert np.all(res["mb_prio"] == 1.0)          # beta = 0
    assert res["offset"] == 200000


def test_importance_weights_closed_form():
    rng = np.random.default_rng(8)
    adv = rng.standard_normal((12, 4)).astype(np.float32)
    res = orp.prio_replay(adv, 0.8, 30, 12, 0.4, seed=9, offset=77)
    assert np.allclose(res["mb_prio"], (12 * res["probs"][res["idx"]].astype(np.float64)) ** -0.4, rtol=1e-6)
    # the stream continues: a second call from the advanced offset draws the next uniforms
    u2 = orp.replay_uniforms(9, 77 + 30, 5)
    assert np.array_equal(u2, orp.replay_uniforms(9, 77, 35)[30:])


def test_index_copy_and_segment_rows():
    dst = np.zeros((6, 3), np.float32)
    src = np.arange(12, dtype=np.float32).reshape(4, 3)
    out = orp.index_copy(dst, np.array([4, 0, 9, -1]), src)
    want = dst.copy()
    want[4], want[0] = src[0], src[1]
    assert np.array_equal(out, want)
    assert np.array_equal(orp.segment_rows([2, 0], 3), [6, 7, 8, 0, 1, 2])


def test_transpose_and_clamp():
    x = np.random.default_rng(10).uniform(-3, 3, (4, 5, 3)).astype(np.float32)
    t = orp.transpose_102(x, clamp=True)
    assert t.shape == (5, 4, 3)
    assert np.array_equal(t[2, 1], np.clip(x[1, 2], -1, 1))
