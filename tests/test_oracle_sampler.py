"""Pins of the oracle's counter RNG and sampler (CPU)."""
import numpy as np
import pytest

import oracle.sampler as S


def test_philox_known_answer_vectors():
    """Philox4x32-10 KATs published with Random123 (kat_vectors)."""
    cases = [
        ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
        ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
        ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
         (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
    ]
    for ctr, key, want in cases:
        got = S.philox4x32_10(np.array([ctr], np.uint32), np.array([key], np.uint32))[0]
        assert tuple(int(x) for x in got) == want


def test_uniforms_are_in_open_interval_and_uniform():
    u = S.uniforms(seed=7, step=3, n=200000)
    assert u.dtype == np.float32 and u.min() > 0 and u.max() < 1
    hist = np.histogram(u, bins=20, range=(0, 1))[0]
    chi2 = ((hist - 10000.0) ** 2 / 10000.0).sum()
    assert chi2 < 45.3   # chi-square 19 dof, p = 0.001
    # streams differ per step and per seed
    assert not np.array_equal(u[:100], S.uniforms(7, 4, 100))
    assert not np.array_equal(u[:100], S.uniforms(8, 3, 100))


def test_single_legal_option_is_always_chosen():
    n, A = 50, 16
    rng = np.random.default_rng(0)
    dec = rng.standard_normal((n, A + 1)).astype(np.float32)
    mask = np.zeros((n, A), np.float32)
    pick = rng.integers(0, A, n)
    mask[np.arange(n), pick] = 1
    acts, lps, vals, _ = S.sample(dec, mask, seed=1, step=0)
    assert np.array_equal(acts, pick)
    assert np.abs(lps).max() < 1e-6
    assert np.array_equal(vals, dec[:, A])


def test_sampling_distribution_matches_softmax():
    A = 8
    logits = np.array([0.5, -1.0, 2.0, 0.0, 1.0, -3.0, 0.3, 1.5], np.float32)
    mask = np.array([1, 1, 1, 0, 1, 1, 1, 1], np.float32)
    n = 40000
    dec = np.tile(np.append(logits, 0.0).astype(np.float32), (n, 1))
    acts, lps, _, _ = S.sample(dec, np.tile(mask, (n, 1)), seed=11, step=5)
    l = np.where(mask == 0, -1e4, logits).astype(np.float64)
    p = np.exp(l - l.max())
    p /= p.sum()
    cnt = np.bincount(acts, minlength=A)
    assert cnt[3] == 0
    keep = p > 0
    chi2 = ((cnt[keep] - n * p[keep]) ** 2 / (n * p[keep])).sum()
    assert chi2 < 24.3   # 6 dof, p = 0.0005
    assert np.allclose(lps, np.log(p[acts]), atol=1e-5)


def test_safe_logits():
    l = S.safe_masked(np.array([np.nan, np.inf, -np.inf, 1.0], np.float32), np.array([1, 1, 1, 0]))
    assert l[0] == 0 and l[1] == np.float32(3.4028e38) and l[2] == np.float32(-3.4028e38) and l[3] == np.float32(-1e4)


# ---- Gumbel-max sampler of the oracle: pinned by float64 math and closed forms

def test_log_rep_against_float64_log():
    """log_rep within 3 ulp of the float64 logarithm over every binade the
    Gumbel transform meets (and well beyond), exact at 1."""
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.random(400000) * np.float32(2.0) ** rng.integers(-30, 30, 400000)).astype(np.float32),
        np.float32(2.0) ** np.arange(-126, 127, dtype=np.float32),
        np.array([1.0, np.nextafter(np.float32(1), np.float32(2)), np.nextafter(np.float32(1), np.float32(0)),
                  1.41421354, 1.41421366, 0.70710677], np.float32)])
    x = x[(x > 0) & np.isfinite(x) & (x >= np.finfo(np.float32).tiny)]
    got = S.log_rep(x).astype(np.float64)
    want = np.log(x.astype(np.float64))
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    ok = want != 0
    assert np.max(np.abs(got - want)[ok] / ulp[ok]) <= 3.0
    assert S.log_rep(np.float32(1.0)) == 0.0


def test_gumbel_noise_distribution_and_layout():
    """g = -log(-log u): mean = Euler's gamma, variance = pi^2 / 6, CDF
    exp(-exp(-g)) (Kolmogorov-Smirnov); the uniforms are the Philox words of
    counter (row, step lo, step hi, 1 + j/4), word j % 4."""
    n, A = 4096, 64
    g = S.gumbel_noise(11, 5, n, A).astype(np.float64).ravel()
    assert abs(g.mean() - 0.5772156649) < 5e-3
    assert abs(g.var() - np.pi ** 2 / 6) < 2e-2
    gs = np.sort(g)
    cdf = np.exp(-np.exp(-gs))
    emp = np.arange(1, gs.size + 1) / gs.size
    assert np.abs(cdf - emp).max() < 1.63 / np.sqrt(gs.size) * 1.5
    u = S.gumbel_uniforms(3, 2 ** 33 + 9, 3, 8)
    w = S.philox4x32_10(np.array([[2, 9, 2, 2]], np.uint64), np.array([[3, 0]], np.uint64))[0]
    want = ((w >> np.uint32(9)).astype(np.float32) * np.float32(2) + np.float32(1)) * np.float32(2.0 ** -24)
    assert np.array_equal(u[2, 4:8], want)


def test_gumbel_max_samples_the_masked_softmax():
    A, n = 10, 200000
    logits = np.linspace(-1.5, 2.0, A).astype(np.float32)
    mask = np.ones(A, np.float32)
    mask[[0, 6]] = 0
    dec = np.tile(np.append(logits, 0).astype(np.float32), (n, 1))
    acts, lps, _ = S.sample_gumbel(dec, np.tile(mask, (n, 1)), S.gumbel_noise(4, 0, n, A))
    l = np.where(mask == 0, -1e4, logits).astype(np.float64)
    p = np.exp(l - l.max())
    p /= p.sum()
    cnt = np.bincount(acts, minlength=A)
    assert cnt[0] == 0 and cnt[6] == 0
    k = p > 1e-9
    assert ((cnt[k] - n * p[k]) ** 2 / (n * p[k])).sum() < 26.1   # 7 dof, p = 0.0005
    assert np.allclose(lps, np.log(p[acts]), atol=1e-12)


def test_gumbel_ties_and_single_legal():
    dec = np.zeros((3, 5), np.float32)
    mask = np.ones((3, 4), np.float32)
    mask[1, :2] = 0
    mask[2] = [0, 0, 1, 0]
    acts, lps, _ = S.sample_gumbel(dec, mask, np.zeros((3, 4), np.float32))
    assert list(acts) == [0, 2, 2]
    assert lps[2] == 0.0
