"""Pins of the oracle's policy forward (CPU).

The reference ships no golden vectors for this path, and its torch model
cannot be built here (it needs the engine SDK), so the oracle restatement is
pinned against independent formulations:
* attention vs torch's F.scaled_dot_product_attention (a library routine);
* the full-length + key-mask forward (the native model's semantics) vs the
  torch model's prefix-sliced formulation (ptcg/rl/model.py:237-262),
  written here as a separate computation, on every live output;
* invariances the masking implies (padded-token contents, batch mates);
* the pointer gather by brute force;
* autograd gradients vs finite differences (gradcheck, fp64).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ptcg_amd import dims, synth
import oracle.model as om

torch.set_num_threads(4)


def test_attention_matches_sdpa():
    torch.manual_seed(0)
    blk = om.Block(32, 4, 64).double()
    x = torch.randn(3, 11, 32, dtype=torch.float64)
    keep = torch.rand(3, 11) < 0.6
    keep[:, 0] = True
    got = blk.attention(x, keep)
    B, L, D = x.shape
    q, k, v = blk.qkv(x).view(B, L, 3, 4, 8).permute(2, 0, 3, 1, 4).unbind(0)
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=keep.view(B, 1, 1, L))
    assert torch.allclose(got, ref.transpose(1, 2).reshape(B, L, D), atol=1e-12)


def _sliced_forward(m, obs):
    """The torch reference's formulation: slice the token axis to the batch's
    longest valid prefix, boolean key mask, pointer gather through a zero-padded
    copy of h (ptcg/rl/model.py:207-276), raw scores (no -1e9 fill)."""
    dm = m.dm
    B, Lt = obs.shape[0], dm.l_tok
    cv, av = m.card_table, m.attack_table
    tok = m._take(obs, "tok_int").reshape(B, Lt, dm.tok_int)
    ti = tok.long()
    cid = ti[:, :, 0].clamp(0, dm.n_cards - 1)
    t0, t1 = ti[:, :, 3], ti[:, :, 4]
    tool = cv[t0.clamp(0, dm.n_cards - 1)] * (t0 > 0).unsqueeze(-1) + \
        cv[t1.clamp(0, dm.n_cards - 1)] * (t1 > 0).unsqueeze(-1)
    x = m.token_proj(torch.cat([cv[cid], tool, m._take(obs, "tok_float").reshape(B, Lt, dm.tok_f),
                                m.zone_emb(ti[:, :, 1].clamp(0, dm.n_zones - 1)),
                                m.owner_emb(ti[:, :, 2].clamp(0, dm.n_owners - 1))], -1))
    g = m.global_mlp(m._take(obs, "global_f"))
    di = m._take(obs, "dec_int").long()
    d_vec = m.dec_mlp(torch.cat([
        m.sel_type_emb(di[:, 0].clamp(0, dm.n_select_types - 1)),
        m.ctx_emb(di[:, 1].clamp(0, dm.n_contexts - 1)),
        cv[di[:, 2].clamp(0, dm.n_cards - 1)], cv[di[:, 3].clamp(0, dm.n_cards - 1)],
        av[di[:, 4].clamp(0, dm.n_attacks - 1)], av[di[:, 5].clamp(0, dm.n_attacks - 1)],
        cv[di[:, 6].clamp(0, dm.n_cards - 1)], cv[di[:, 7].clamp(0, dm.n_cards - 1)],
        m._take(obs, "dec_float")], -1))
    x = x + m.bcast(torch.cat([g, d_vec], -1)).unsqueeze(1)
    valid = ti[:, :, 1] > 0
    L = int(valid.sum(1).max())
    x = torch.cat([m.readout.expand(B, 1, -1), x[:, :L]], 1)
    keep = torch.cat([torch.ones(B, 1, dtype=torch.bool), valid[:, :L]], 1).view(B, 1, 1, -1)
    for blk in m.blocks:
        h1 = blk.ln1(x)
        q, k, v = blk.qkv(h1).view(B, L + 1, 3, blk.heads, dm.d // blk.heads).permute(2, 0, 3, 1, 4).unbind(0)
        a = F.scaled_dot_product_attention(q, k, v, attn_mask=keep)
        x = x + blk.proj(a.transpose(1, 2).reshape(B, L + 1, dm.d))
        x = x + blk.ffn(blk.ln2(x))
    h = m.ln_f(x)
    r = h[:, 0]
    oi = m._take(obs, "opt_int").reshape(B, dm.n_opt, dm.opt_int).long()
    hz = torch.zeros(B, Lt + 1, dm.d, dtype=h.dtype)
    hz[:, 1:L + 1] = h[:, 1:]
    p1 = hz.gather(1, oi[:, :, 1].clamp(0, Lt).unsqueeze(-1).expand(-1, -1, dm.d))
    p2 = hz.gather(1, oi[:, :, 2].clamp(0, Lt).unsqueeze(-1).expand(-1, -1, dm.d))
    q = m.q_mlp(torch.cat([m.opt_type_emb(oi[:, :, 0].clamp(0, dm.n_opt_types - 1)), p1, p2,
                           m.opt_card(cv[oi[:, :, 3].clamp(0, dm.n_cards - 1)]),
                           m.opt_attack(av[oi[:, :, 4].clamp(0, dm.n_attacks - 1)]),
                           m._take(obs, "opt_float").reshape(B, dm.n_opt, dm.opt_f)], -1))
    rr = r.unsqueeze(1).expand(-1, dm.n_opt, -1)
    scores = m.score_mlp(torch.cat([q, rr, g.unsqueeze(1).expand(-1, dm.n_opt, -1),
                                    d_vec.unsqueeze(1).expand(-1, dm.n_opt, -1), q * rr], -1)).squeeze(-1)
    value = m.value_mlp(torch.cat([r, g], -1))
    return torch.cat([scores, value], -1)


@pytest.mark.parametrize("dm", [dims.tiny(), dims.tiny(heads=1, d=32, ffn=64)], ids=["tiny", "tiny_h1"])
def test_full_length_masked_forward_equals_prefix_sliced(dm):
    m = om.build(dm, seed=4, dtype=torch.float64)
    obs = torch.from_numpy(synth.make_obs(dm, 9, seed=5)).double()
    with torch.no_grad():
        a = m(obs)
        b = _sliced_forward(m, obs)
    assert torch.allclose(a, b, atol=1e-10, rtol=1e-10)


def test_padded_token_contents_do_not_matter():
    dm = dims.tiny()
    m = om.build(dm, seed=6, dtype=torch.float64)
    obs = synth.make_obs(dm, 6, seed=7)
    off = dm.offsets()
    obs2 = obs.copy()
    ti = obs2[:, off["tok_int"][0]:off["tok_int"][1]].reshape(6, dm.l_tok, dm.tok_int)
    tf = obs2[:, off["tok_float"][0]:off["tok_float"][1]].reshape(6, dm.l_tok, dm.tok_f)
    pad = ti[:, :, 1] == 0
    assert pad.any()
    rng = np.random.default_rng(0)
    tf[pad] = rng.standard_normal((pad.sum(), dm.tok_f))
    ti[pad, 0] = rng.integers(0, dm.n_cards, pad.sum())
    with torch.no_grad():
        a = m(torch.from_numpy(obs).double())
        b = m(torch.from_numpy(obs2).double())
    assert torch.allclose(a, b, atol=1e-12)


def test_batch_independence():
    dm = dims.tiny()
    m = om.build(dm, seed=8, dtype=torch.float64)
    obs = torch.from_numpy(synth.make_obs(dm, 7, seed=9, rich=True)).double()
    with torch.no_grad():
        full = m(obs)
        single = torch.cat([m(obs[i:i + 1]) for i in range(7)])
    assert torch.allclose(full, single, atol=1e-12)


def test_pointer_gather_brute_force():
    dm = dims.tiny()
    m = om.build(dm, seed=10, dtype=torch.float64)
    obs_np = synth.make_obs(dm, 4, seed=11, rich=True)
    off = dm.offsets()
    oi = obs_np[:, off["opt_int"][0]:off["opt_int"][1]].reshape(4, dm.n_opt, dm.opt_int)
    oi[0, 0, 1] = dm.l_tok + 3     # out of range -> zeros (native rule)
    oi[0, 1, 1] = -2
    obs = torch.from_numpy(obs_np).double()
    with torch.no_grad():
        out, parts = m(obs, return_parts=True)
        h = parts["h"]
        # rebuild q_mlp's pointer inputs element by element
        for n in range(4):
            for j in range(dm.n_opt):
                for which in (1, 2):
                    p = int(oi[n, j, which])
                    want = h[n, p] if 0 < p <= dm.l_tok else torch.zeros(dm.d, dtype=h.dtype)
                    got_idx = (torch.tensor(p).clamp(0, dm.l_tok))
                    ok = 0 < p <= dm.l_tok
                    got = h[n, got_idx] * ok
                    assert torch.equal(got, want)


def test_autograd_matches_finite_differences():
    dm = dims.tiny(l_tok=5, n_opt=4, d=8, heads=2, ffn=16, d_c=8, d_a=4, g=8, layers=1,
                   n_cards=11, n_attacks=7, tok_f=4)
    m = om.build(dm, seed=12, dtype=torch.float64)
    obs = torch.from_numpy(synth.make_obs(dm, 3, seed=13, rich=True)).double()
    names = ["card_table", "blocks.0.qkv.weight", "score_mlp.0.bias", "readout", "blocks.0.ln1.weight", "q_mlp.0.bias"]
    params = dict(m.named_parameters())
    base = {k: v.detach().clone() for k, v in params.items()}

    def f(*ts):
        p = dict(base)
        p.update(dict(zip(names, ts)))
        out = torch.func.functional_call(m, p, (obs,))
        w = torch.linspace(-1, 1, out.numel(), dtype=out.dtype).view_as(out)
        return (out * w).sum()

    inputs = tuple(base[n].clone().requires_grad_() for n in names)
    assert torch.autograd.gradcheck(f, inputs, eps=1e-6, atol=1e-6, rtol=1e-4)


def test_blob_round_trip():
    dm = dims.tiny()
    m = om.build(dm, seed=14)
    blob = m.to_blob()
    m2 = om.build(dm, seed=99)
    m2.load_blob(blob)
    assert np.array_equal(m2.to_blob(), blob)
    with pytest.raises(ValueError, match="blob has"):
        m2.load_blob(np.zeros(blob.size + 1, np.float32))


# ---------------------------------------------------------------- static tables, oracle critic, aux losses
def _frozen(seed=0, dtype=torch.float64, **kw):
    dm = dims.tiny_frozen(**kw)
    st = synth.make_static(dm, seed + 100)
    return dm, st, om.build(dm, seed=seed, dtype=dtype, static=st)


def test_static_tables_brute_force():
    """CardVec / AttackVec against element-wise loops of the native kernels
    k_att_in, k_sk_in, k_pool, k_card_in (ptcg_model.cu:218-286)."""
    dm, st, m = _frozen(seed=1)
    with torch.no_grad():
        cv, av = m.tables()
        W = lambda mod: (mod.weight.numpy(), mod.bias.numpy())
        gelu = lambda x: 0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2)))
        aw, ab = W(m.attack_mlp[0])
        att = gelu(np.concatenate([m.attack_id_emb.weight.numpy(), st["att_static"], st["att_text"]], 1) @ aw.T + ab)
        assert np.allclose(av.numpy(), att, atol=1e-12)
        sw, sb = W(m.skill_mlp[0])
        sk = gelu(np.concatenate([m.skill_id_emb.weight.numpy(), st["skill_text"]], 1) @ sw.T + sb)
        for c in range(dm.n_cards):
            def pool(tab, ids):
                vals = [tab[i] if i > 0 else np.zeros(tab.shape[1]) for i in ids]
                n = sum(1 for i in ids if i > 0)
                mean = sum(v for i, v in zip(ids, vals) if i > 0) / max(n, 1) if n else np.zeros(tab.shape[1])
                return mean, np.max(np.stack(vals), 0)
            am, ax = pool(att, st["card_attacks"][c])
            sm, sx = pool(sk, st["card_skills"][c])
            ci = np.concatenate([m.card_id_emb.weight[c].numpy(), st["card_static"][c], st["card_text"][c],
                                 am, ax, sm, sx])
            ln = m.card_mlp[0]
            x = (ci - ci.mean()) / math.sqrt(ci.var() + 1e-5) * ln.weight.numpy() + ln.bias.numpy()
            w1, b1 = W(m.card_mlp[1])
            w3, b3 = W(m.card_mlp[3])
            want = gelu(x @ w1.T + b1) @ w3.T + b3
            assert np.allclose(cv[c].numpy(), want, atol=1e-10), c


def test_max_pool_gradient_goes_to_first_maximal_slot():
    v = torch.tensor([[[1.0, 2.0], [3.0, 2.0], [3.0, 0.5]]], dtype=torch.float64, requires_grad=True)
    om.first_max_pool(v).sum().backward()
    # column 0: tie between slots 1 and 2 -> slot 1; column 1: tie between slots 0 and 1 -> slot 0
    assert v.grad[0, :, 0].tolist() == [0.0, 1.0, 0.0]
    assert v.grad[0, :, 1].tolist() == [1.0, 0.0, 0.0]


def test_oracle_critic_equals_torch_prefix_formulation():
    """The critic over the full-length trunk (native) gives the value of the
    torch model's prefix-sliced critic (model.py:278-308) on every row."""
    dm, st, m = _frozen(seed=2)
    obs = torch.from_numpy(synth.make_obs(dm, 6, seed=3, rich=True)).double()
    with torch.no_grad():
        out, parts = m(obs, return_parts=True)
        h, keep, g, cv = parts["h"], parts["keep"], parts["g"], parts["card_vec"]
        B = obs.shape[0]
        L = int(keep[:, 1:].sum(1).max())
        hand, split, prize = m._oracle_ids(obs)
        ids = torch.cat([hand[:, :, 0], split[:, :, 0], prize[:, :, 0]], 1).long().clamp(0, dm.n_cards - 1)
        feats = torch.zeros(B, 56, 6, dtype=torch.float64)
        feats[:, :24, 0] = 1
        feats[:, :24, 3] = hand[:, :, 1]
        feats[:, 24:48, 1] = 1
        feats[:, 24:48, 4] = split[:, :, 1]
        feats[:, 24:48, 5] = split[:, :, 2]
        feats[:, 48:, 2] = 1
        feats[:, 48:, 3] = prize[:, :, 1]
        otok = m.oracle_proj(torch.cat([cv[ids], feats], -1))
        x = torch.cat([m.critic_readout.expand(B, 1, -1), h[:, :L + 1], otok], 1)
        one = torch.ones(B, 1, dtype=torch.bool)
        kc = torch.cat([one, one, keep[:, 1:L + 1], ids > 0], 1)
        blk = m.critic_blocks[0]
        hh = blk.ln1(x)
        q, k, v = blk.qkv(hh).view(B, x.shape[1], 3, blk.heads, dm.d // blk.heads).permute(2, 0, 3, 1, 4).unbind(0)
        a = F.scaled_dot_product_attention(q, k, v, attn_mask=kc.view(B, 1, 1, -1))
        x = x + blk.proj(a.transpose(1, 2).reshape(B, x.shape[1], dm.d))
        x = x + blk.ffn(blk.ln2(x))
        want = m.oracle_value_mlp(torch.cat([x[:, 0], g], -1)).squeeze(-1)
    assert torch.allclose(out[:, -1], want, atol=1e-10)


def test_aux_loss_gradients_match_the_native_formulas():
    """d/d(parts) of aux_loss equals k_blind_grad / k_hand_grad / k_prize_grad
    (ptcg_model2.cu:243-287) written out in closed form."""
    dm, st, m = _frozen(seed=4)
    obs_np = synth.make_obs(dm, 7, seed=5, rich=True)
    obs = torch.from_numpy(obs_np).double()
    ret = np.random.default_rng(6).standard_normal(7)
    with torch.no_grad():
        _, parts = m(obs, return_parts=True)
    leaf = {k: parts[k].clone().requires_grad_() for k in ("blind_v", "hand_lin", "prize_logit")}
    p2 = dict(parts, **leaf)
    m.aux_loss(obs, p2, ret).backward()
    N, NC, Lt = 7, dm.n_cards, dm.l_tok
    off = dm.offsets()
    o = obs_np[:, off["oracle"][0]:off["oracle"][1]]
    tgt = np.zeros((N, NC))
    prized = np.zeros((N, NC))
    for n in range(N):
        for k in range(24):
            i, c = int(o[n, 2 * k]), o[n, 2 * k + 1] * 4.0
            if 0 < i < NC and i != NC - 1 and c != 0:
                tgt[n, i] += c
        for s in range(8):
            i, c = int(o[n, 120 + 2 * s]), o[n, 121 + 2 * s]
            if 0 < i < NC and c > 0:
                prized[n, i] = 1.0
    x = parts["hand_lin"].numpy()
    sp = np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))
    sig = 1 / (1 + np.exp(-x))
    assert np.allclose(leaf["hand_lin"].grad.numpy(), 0.1 * 2 * (sp - tgt) / (N * NC) * np.where(x > 20, 1, sig),
                       atol=1e-14)
    assert np.allclose(leaf["blind_v"].grad.numpy().ravel(), (parts["blind_v"].numpy().ravel() - ret) / N, atol=1e-14)
    ti = obs_np[:, off["tok_int"][0]:off["tok_int"][1]].reshape(N, Lt, dm.tok_int)
    unseen = ti[:, :, 1].astype(np.int64) == 9
    assert unseen.any()
    cnt = unseen.sum()
    lg = parts["prize_logit"].numpy()
    cid = np.clip(ti[:, :, 0].astype(np.int64), 0, NC - 1)
    t = np.take_along_axis(prized, cid, 1)
    want = np.where(unseen, 0.1 * (1 / (1 + np.exp(-lg)) - t) / cnt, 0.0)
    assert np.allclose(leaf["prize_logit"].grad.numpy(), want, atol=1e-14)


def test_frozen_variant_autograd_matches_finite_differences():
    dm, st, m = _frozen(seed=7, l_tok=5, n_opt=4, d=8, heads=2, ffn=16, d_c=8, d_a=4, g=8, layers=1,
                        n_cards=11, n_attacks=7, n_skills=5, tok_f=4)
    obs = torch.from_numpy(synth.make_obs(dm, 3, seed=8, rich=True)).double()
    ret = torch.tensor([0.3, -1.0, 0.7], dtype=torch.float64)
    # small tensors from every new stage (gradcheck perturbs each element)
    names = ["attack_mlp.0.bias", "skill_id_emb.weight", "card_mlp.0.weight", "card_mlp.3.bias",
             "oracle_proj.bias", "critic_readout", "critic_blocks.0.ln1.weight", "aux_hand.bias",
             "aux_prize.weight", "value_mlp.2.weight"]
    base = {k: v.detach().clone() for k, v in m.named_parameters()}

    def f(*ts):
        p = dict(base)
        p.update(dict(zip(names, ts)))
        out, parts = torch.func.functional_call(m, p, (obs,), {"return_parts": True})
        w = torch.linspace(-1, 1, out.numel(), dtype=out.dtype).view_as(out)
        return (out * w).sum() + m.aux_loss(obs, parts, ret)

    inputs = tuple(base[n].clone().requires_grad_() for n in names)
    assert torch.autograd.gradcheck(f, inputs, eps=1e-6, atol=1e-6, rtol=1e-4)
