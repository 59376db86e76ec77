"""Counter-based action sampler (oracle; test infrastructure).

* RNG: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers:
  as easy as 1, 2, 3", SC'11), restated from the paper: 10 rounds of
  (hi, lo) = mulhilo(M, c) with M0 = 0xD2511F53, M1 = 0xCD9E8D57 and the
  Weyl key bumps W0 = 0x9E3779B9, W1 = 0xBB67AE85.  Pinned by the
  published known-answer vectors (tests/test_oracle_sampler.py).
  Keying: counter = (row, step low, step high, 0), key = (seed low, seed
  high); the reference instead keeps one advancing cuRAND state per row
  (pufferlib.cu:511-516,614,717) — a counter RNG gives every (seed, step,
  row) its own stream without state in memory.
* uniform: u = (2 (x0 >> 9) + 1) * 2^-24, exactly representable in fp32,
  in [2^-24, 1 - 2^-24].
* sampling: the reference's discrete head (sample_logits,
  pufferlib.cu:584-718): logits made safe (NaN -> 0, +-inf -> +-3.4028e38),
  masked options -> -1e4, online max / sum-exp, inverse-CDF walk over
  exp(l - logsumexp), fallback to the last legal option when rounding leaves
  the CDF below u; logprob = l[a] - logsumexp; value = the fused last column.
  Restated in float32 arithmetic in the same order.
* Gumbel-max (no counterpart in the reference): a = argmax_j (l_j + g_j),
  ties to the lowest j, g_j = -log(-log u_j), u_j from Philox4x32-10 with
  counter (row, step lo, step hi, 1 + j/4), word j % 4.  ``log_rep`` is the
  product's logarithm: argument reduction to m in [sqrt(1/2), sqrt(2)) and
  the atanh series log m = 2 s (1 + z/3 + ... + z^5/11), s = (m-1)/(m+1),
  z = s^2 (Abramowitz & Stegun 4.1.27), evaluated here with numpy float32
  operations in the kernel's order, each correctly rounded, so the noise
  and the draws agree bit for bit.
"""
import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr, key):
    """ctr: (..., 4) uint32, key: (..., 2) uint32 -> (..., 4) uint32."""
    c = [np.asarray(ctr[..., i], dtype=np.uint64) for i in range(4)]
    k0 = np.asarray(key[..., 0], dtype=np.uint64)
    k1 = np.asarray(key[..., 1], dtype=np.uint64)
    for _ in range(10):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK32
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        k0 = (k0 + np.uint64(W0)) & MASK32
        k1 = (k1 + np.uint64(W1)) & MASK32
    return np.stack([x.astype(np.uint32) for x in c], -1)


def uniforms(seed, step, n):
    """One uniform per row 0..n-1 for (seed, step)."""
    rows = np.arange(n, dtype=np.uint64)
    ctr = np.stack([rows, np.full(n, step & 0xFFFFFFFF, np.uint64), np.full(n, (step >> 32) & 0xFFFFFFFF, np.uint64),
                    np.zeros(n, np.uint64)], -1)
    key = np.broadcast_to(np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], np.uint64), (n, 2))
    x = philox4x32_10(ctr, key)[:, 0]
    return ((x >> np.uint32(9)).astype(np.float32) * np.float32(2) + np.float32(1)) * np.float32(2.0 ** -24)


def safe_masked(logits, mask):
    l = np.asarray(logits, dtype=np.float32).copy()
    l[np.isnan(l)] = 0.0
    l[np.isposinf(l)] = np.float32(3.4028e38)
    l[np.isneginf(l)] = np.float32(-3.4028e38)
    l[np.asarray(mask) == 0] = np.float32(-1e4)
    return l


def sample_row(l, u, mask):
    """The reference's inverse-CDF walk on one row of safe, masked logits (fp32)."""
    f = np.float32
    mx, se = f(-np.inf), f(0.0)
    for v in l:
        if v > mx:
            se = se * np.exp(f(mx - v), dtype=np.float32)
            mx = v
        se = se + np.exp(f(v - mx), dtype=np.float32)
    lse = f(mx + np.log(se, dtype=np.float32))
    cs, a = f(0.0), -1
    for j, v in enumerate(l):
        cs = f(cs + np.exp(f(v - lse), dtype=np.float32))
        if u < cs:
            a = j
            break
    if a < 0:
        legal = np.flatnonzero(np.asarray(mask) != 0)
        a = int(legal[-1]) if legal.size else len(l) - 1
    return a, f(l[a] - lse), lse


def sample(dec_out, mask, seed, step):
    """dec_out (n, A+1) = [scores || value], mask (n, A) -> actions (n,),
    logprobs (n,), values (n,), and the uniforms used."""
    dec_out = np.asarray(dec_out, dtype=np.float32)
    n, A1 = dec_out.shape
    A = A1 - 1
    u = uniforms(seed, step, n)
    acts = np.zeros(n, np.int64)
    lps = np.zeros(n, np.float32)
    for i in range(n):
        l = safe_masked(dec_out[i, :A], mask[i])
        acts[i], lps[i], _ = sample_row(l, u[i], mask[i])
    return acts, lps, dec_out[:, A].copy(), u


def boundary_margin(dec_out, mask, u):
    """float64 distance of each row's uniform from the nearest CDF step —
    rows where fp32 rounding may legitimately pick the neighbouring option."""
    dec_out = np.asarray(dec_out, dtype=np.float64)
    A = dec_out.shape[1] - 1
    out = np.zeros(len(u))
    for i in range(len(u)):
        l = safe_masked(dec_out[i, :A], mask[i]).astype(np.float64)
        p = np.exp(l - l.max())
        cdf = np.cumsum(p / p.sum())
        out[i] = np.abs(cdf - float(u[i])).min()
    return out


# ---- Gumbel-max
_F = np.float32
LOG_C = [_F(1 / 11), _F(1 / 9), _F(1 / 7), _F(1 / 5), _F(1 / 3)]
LN2_HI = _F(0.693145751953125)                  # 0x3f317200: e * LN2_HI is exact
LN2_LO = _F(np.log(2.0) - 0.693145751953125)    # 0x35bfbe8e


def log_rep(x):
    """log of positive normal float32 values, in the kernel's exact fp32 order."""
    x = np.asarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.int64)
    e = (b >> 23) - 127
    mb = (b & 0x007FFFFF) | 0x3F800000
    big = mb > 0x3FB504F3
    mb = np.where(big, mb - 0x00800000, mb)
    e = np.where(big, e + 1, e)
    m = mb.astype(np.uint32).view(np.float32)
    s = (m - _F(1)) / (m + _F(1))
    z = s * s
    p = np.full_like(z, LOG_C[0])
    for c in LOG_C[1:]:
        p = c + z * p
    p = _F(1) + z * p
    lm = (s + s) * p
    ef = e.astype(np.float32)
    return ef * LN2_HI + (lm + ef * LN2_LO)


def gumbel_uniforms(seed, step, n, A):
    """u (n, A): Philox4x32-10 counter (row, step lo, step hi, 1 + j/4), word j % 4."""
    groups = (A + 3) // 4
    rows = np.repeat(np.arange(n, dtype=np.uint64), groups)
    grp = np.tile(np.arange(groups, dtype=np.uint64), n) + np.uint64(1)
    m = rows.size
    ctr = np.stack([rows, np.full(m, step & 0xFFFFFFFF, np.uint64),
                    np.full(m, (step >> 32) & 0xFFFFFFFF, np.uint64), grp], -1)
    key = np.broadcast_to(np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], np.uint64), (m, 2))
    x = philox4x32_10(ctr, key).reshape(n, groups * 4)[:, :A]
    return ((x >> np.uint32(9)).astype(np.float32) * np.float32(2) + np.float32(1)) * np.float32(2.0 ** -24)


def gumbel_noise(seed, step, n, A):
    return -log_rep(-log_rep(gumbel_uniforms(seed, step, n, A)))


def sample_gumbel(dec_out, mask, noise):
    """dec_out (n, A+1), mask (n, A), noise (n, A) -> actions (n,) int,
    logprobs (n,) (float64 log-softmax of the draw), values (n,)."""
    dec_out = np.asarray(dec_out, dtype=np.float32)
    n, A1 = dec_out.shape
    A = A1 - 1
    l = np.stack([safe_masked(dec_out[i, :A], mask[i]) for i in range(n)])
    v = l + np.asarray(noise, dtype=np.float32)          # fp32 adds
    acts = np.argmax(v, axis=1)                           # first maximum
    l64 = l.astype(np.float64)
    lse = l64.max(1) + np.log(np.exp(l64 - l64.max(1, keepdims=True)).sum(1))
    lps = l64[np.arange(n), acts] - lse
    return acts, lps, dec_out[:, A].copy()
