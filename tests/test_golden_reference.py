"""The oracle and the product's tables against the reference's own torch model.

The golden vectors (tests/golden/reference_*.npz) were written by
``make_reference_fixtures.py`` from ``PTCGTransformer.forward_train`` /
``forward_eval`` (ptcg/rl/model.py:207-341) and ``native_weights.param_order``
/ ``blob_to_sd`` (native/tools/native_weights.py:45-113).  They pin what no
closed form does: the blob's full tensor order and the model's wiring (token,
decision, q and score concat orders, pointer targets, head inputs, oracle-token
features, aux heads).  Planted mistakes in the oracle's inputs / weights
(same-shape tensors swapped, two same-width concat blocks swapped, Q and K
swapped) must fail these checks.

Tolerances: the oracle runs in float64, the reference ran in float32 —
outputs relative L2 <= 1e-5 and max|d| <= 1e-4 * max(1, max|ref|); gradient
summaries within 1e-4 of each tensor's norm (refvec.Fixture.grad_check).
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from refvec import CASES, load
from ptcg_amd import params
import oracle.layout as olayout
import oracle.model as om


def _oracle_outputs(fx, blob=None, obs=None):
    ref = om.build(fx.dm, blob=fx.blob if blob is None else blob, dtype=torch.float64, static=fx.static)
    o = torch.from_numpy(fx.obs if obs is None else obs).double()
    out, parts = ref(o, return_parts=True)
    L = fx.L
    res = dict(logits=out[:, :fx.dm.n_opt], oracle_v=out[:, fx.dm.n_opt:], blind_v=parts["blind_v"],
               hand_pred=torch.nn.functional.softplus(parts["hand_lin"]),
               prize_logits=parts["prize_logit"][:, :L])
    return ref, res


def _objective(fx, res, which):
    z = fx.z
    legal = torch.from_numpy(fx.legal())
    w = {k: torch.from_numpy(z[f"w_{k}"]).double()
         for k in ("logits", "oracle_v", "blind_v", "hand_pred", "prize_logits")}
    obj = (torch.where(legal, res["logits"], torch.zeros_like(res["logits"])) * w["logits"]).sum() \
        + (res["oracle_v"] * w["oracle_v"]).sum()
    if which == "A":
        obj = obj + sum((res[k] * w[k]).sum() for k in ("blind_v", "hand_pred", "prize_logits"))
    return obj


def _compare_forward(fx, res):
    z = fx.z
    legal = fx.legal()
    got = res["logits"].detach().numpy()
    errs = {"logits": (got[legal], z["logits"][legal])}
    for k in ("oracle_v", "blind_v", "hand_pred", "prize_logits"):
        errs[k] = (res[k].detach().numpy(), z[k])
    out = {}
    for k, (a, b) in errs.items():
        scale = max(1.0, float(np.abs(b).max()))
        out[k] = (rel_l2(a, b), float(np.abs(a - b).max()) / scale)
    return out


@pytest.fixture(scope="module", params=CASES)
def fx(request):
    return load(request.param)


def test_blob_order_is_the_references(fx):
    """params.param_order / oracle.layout.blob_order == native_weights.param_order, entry by entry."""
    want = list(zip(fx.names, fx.shapes))
    got = [(n, tuple(s)) for n, s in params.param_order(fx.dm)]
    assert got == want
    assert [(n, tuple(s)) for n, s in olayout.blob_order(fx.dm)] == want
    assert params.packed_size(fx.dm) == fx.blob.size


def test_fixture_inputs(fx):
    """The fixture's own invariants: the reference's prefix length, legal-only
    logits (illegal filled with -1e9), forward_eval under critic='blind' ==
    the blind value head of forward_train."""
    z = fx.z
    dm = fx.dm
    t0, _ = dm.offsets()["tok_int"]
    zone = fx.obs[:, t0:t0 + dm.l_tok * dm.tok_int].reshape(-1, dm.l_tok, dm.tok_int)[:, :, 1]
    assert fx.L == int((zone.astype(np.int64) > 0).sum(1).max())
    assert np.all(z["logits"][~fx.legal()] == np.float32(-1e9))
    np.testing.assert_array_equal(z["eval_blind_v"], z["blind_v"])


def test_oracle_forward_matches_reference(fx):
    _, res = _oracle_outputs(fx)
    errs = _compare_forward(fx, res)
    for k, (r, m) in errs.items():
        assert r <= 1e-5 and m <= 1e-4, (k, r, m)


@pytest.mark.parametrize("which", ["A", "C"])
def test_oracle_gradients_match_reference(fx, which):
    ref, res = _oracle_outputs(fx)
    _objective(fx, res, which).backward()
    grads = {n: (p.grad if p.grad is not None else torch.zeros_like(p)).numpy()
             for n, p in ref.named_blob_params()}
    bad = fx.grad_check(which, grads)
    assert not bad, bad[:8]


# ---- planted mistakes: each must move the outputs well past the tolerance

def _max_forward_err(fx, **kw):
    _, res = _oracle_outputs(fx, **kw)
    return max(max(v) for v in _compare_forward(fx, res).values())


def test_planted_blob_swap_is_detected(fx):
    """ln1.weight <-> ln1.bias and qkv's Q <-> K row blocks of block 0."""
    order = params.param_order(fx.dm)
    offs = np.cumsum([0] + [int(np.prod(s)) for _, s in order])
    idx = {n: i for i, (n, _) in enumerate(order)}
    blob = fx.blob.copy()
    a, b = idx["blocks.0.ln1.weight"], idx["blocks.0.ln1.bias"]
    blob[offs[a]:offs[a + 1]], blob[offs[b]:offs[b + 1]] = fx.blob[offs[b]:offs[b + 1]], fx.blob[offs[a]:offs[a + 1]]
    assert _max_forward_err(fx, blob=blob) > 1e-2
    blob = fx.blob.copy()
    q = idx["blocks.0.qkv.weight"]
    w = blob[offs[q]:offs[q + 1]].reshape(3, fx.dm.d, fx.dm.d)
    w[[0, 1]] = w[[1, 0]]
    assert _max_forward_err(fx, blob=blob) > 1e-2


def test_planted_concat_swap_is_detected(fx):
    """Two same-width decision-input blocks (the effect and context CardVecs,
    dec_int columns 2 and 3) swapped."""
    obs = fx.obs.copy()
    d0, _ = fx.dm.offsets()["dec_int"]
    obs[:, [d0 + 2, d0 + 3]] = obs[:, [d0 + 3, d0 + 2]]
    assert np.any(obs[:, d0 + 2] != obs[:, d0 + 3])
    assert _max_forward_err(fx, obs=obs) > 1e-3
