"""PyTorch CPU restatement of the policy forward (oracle; test infrastructure).

Follows ptcg/rl/model.py:70-341 module for module, with the NATIVE model's
semantics where the two differ (native/model/ptcg_model*.cu is the path the
build replaces):

* the trunk runs the full ``l_tok + 1`` positions with a key mask
  (ptcg_model3.cu:12-40) instead of slicing to the batch's longest valid
  prefix (model.py:237-244); keep = zone_float > 0 on the raw fp32 zone
  (ptcg_model.cu:360-367), position 0 (READOUT) always kept;
* masked keys score -1e30 before the softmax (ptcg_kernels.cuh:223-236);
* the option scores leave the model RAW (no -1e9 fill, model.py:274);
  masking happens in the loss at -1e4 (pufferlib.cu:949-962);
* pointer ids p outside (0, l_tok] read a zero vector (ptcg_model.cu:405-411);
* ids are fp32 truncated toward zero then clamped (ptcg_model.cu:299-318),
  which ``Tensor.long()`` + ``clamp`` reproduces.

Output is the decoder contract (N, n_opt + 1) = [raw scores || value]
(ptcg_model.cu:512-517).  Two variants per switch:

* tables: learned (n_cards, d_c) / (n_attacks, d_a) tables (the synthetic
  workload), or the reference's static-table chain (model.py:185-205,
  ptcg_model2.cu:422-485) rebuilt every forward from uploaded static
  features: AttackVec = GELU(Linear([id48 | static15 | text64])), SkillVec
  likewise, CardVec = MLP(LN([id64 | static58 | text128 | attack mean/max |
  skill mean/max])).  The max pool follows the native kernel (k_pool,
  ptcg_model.cu:236-256): masked slots take part as 0 and the gradient goes
  to the FIRST maximal slot (torch's amax would split it between ties);
* critic: blind (value = value_mlp([r | g])) or the oracle critic block
  over [critic readout | h | 56 oracle tokens] (model.py:278-308,
  ptcg_model.cu:442-509) whose value fills the output column, with the
  blind value head and the belief aux heads trained by the aux losses the
  native backward injects (ptcg_model4.cu:26-61, ptcg_model2.cu:219-285):
  blind-V MSE (coef 1), softplus hand-count MSE (0.1), per-MY_UNSEEN-token
  prize BCE (0.1).  :func:`aux_loss` states them as one differentiable
  objective whose autograd gradient is the kernels' gradient.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .layout import offsets, blob_order

# static feature widths and pool fan-ins of the reference tables
# (ptcg/rl/cards.py:19-82; ptcg_model2.cu:383-396)
STATIC_SHAPES = dict(card_static=58, att_static=15, card_text=128, att_text=64, skill_text=64)
K_ATT, K_SK = 4, 2
# oracle block: 24 opp-hand (id, count/4), 24 split (id, deck/4, prize/4),
# 8 my-prize (id, count/4) slots (ptcg/rl/buffers.py:42-45)
N_HAND, N_SPLIT, N_PRIZE = 24, 24, 8
ZONE_MY_UNSEEN = 9
AUX_VF_COEF, AUX_HAND_COEF, AUX_PRIZE_COEF = 1.0, 0.1, 0.1   # ptcg_model.cu:85-87


def card_in_width(dm):
    """[id64 | static58 | text128 | a_mean | a_max | s_mean | s_max]"""
    return 64 + 58 + 128 + 2 * dm.d_a + 2 * dm.d_c


class Block(nn.Module):
    """Pre-LN block (model.py:70-91; ptcg_model3.cu:12-40)."""

    def __init__(self, d, heads, ffn):
        super().__init__()
        self.heads = heads
        self.ln1 = nn.LayerNorm(d)
        self.qkv = nn.Linear(d, 3 * d)
        self.proj = nn.Linear(d, d)
        self.ln2 = nn.LayerNorm(d)
        self.ffn = nn.Sequential(nn.Linear(d, ffn), nn.GELU(), nn.Linear(ffn, d))

    def attention(self, x, keep):
        B, L, D = x.shape
        H = self.heads
        q, k, v = self.qkv(x).view(B, L, 3, H, D // H).permute(2, 0, 3, 1, 4).unbind(0)
        s = torch.matmul(q, k.transpose(-1, -2)) * (1.0 / math.sqrt(D // H))
        s = s.masked_fill(~keep[:, None, None, :], -1e30)
        p = torch.softmax(s, dim=-1)
        a = torch.matmul(p, v)
        return a.transpose(1, 2).reshape(B, L, D)

    def forward(self, x, keep):
        x = x + self.proj(self.attention(self.ln1(x), keep))
        return x + self.ffn(self.ln2(x))


def first_max_pool(v):
    """max over dim 1 whose gradient goes to the first maximal slot only."""
    idx = torch.argmax(v, dim=1, keepdim=True)
    return v.gather(1, idx).squeeze(1)


class OraclePolicy(nn.Module):
    def __init__(self, dm):
        super().__init__()
        self.dm = dm
        d, dc, da, G = dm.d, dm.d_c, dm.d_a, dm.g
        self.off, self.obs_size = offsets(dm)
        if dm.tables == 0:
            self.card_table = nn.Parameter(torch.randn(dm.n_cards, dc))
            self.attack_table = nn.Parameter(torch.randn(dm.n_attacks, da))
        else:
            self.card_id_emb = nn.Embedding(dm.n_cards, 64)
            self.attack_id_emb = nn.Embedding(dm.n_attacks, 48)
            self.skill_id_emb = nn.Embedding(dm.n_skills, 48)
            self.attack_mlp = nn.Sequential(nn.Linear(48 + 15 + 64, da), nn.GELU())
            self.skill_mlp = nn.Sequential(nn.Linear(48 + 64, dc), nn.GELU())
            ci = card_in_width(dm)
            self.card_mlp = nn.Sequential(nn.LayerNorm(ci), nn.Linear(ci, 256), nn.GELU(), nn.Linear(256, dc))
            self.static = None
        self.zone_emb = nn.Embedding(dm.n_zones, 8)
        self.owner_emb = nn.Embedding(dm.n_owners, 4)
        self.token_proj = nn.Linear(2 * dc + dm.tok_f + 8 + 4, d)
        self.readout = nn.Parameter(torch.randn(d) * 0.02)
        self.global_mlp = nn.Sequential(nn.Linear(dm.global_f, G), nn.GELU(), nn.Linear(G, G))
        self.sel_type_emb = nn.Embedding(dm.n_select_types, 8)
        self.ctx_emb = nn.Embedding(dm.n_contexts, 32)
        dec_in = 8 + 32 + 2 * dc + 2 * da + 2 * dc + dm.dec_f
        self.dec_mlp = nn.Sequential(nn.Linear(dec_in, 64), nn.GELU(), nn.Linear(64, 64))
        self.bcast = nn.Linear(G + 64, d)
        self.blocks = nn.ModuleList(Block(d, dm.heads, dm.ffn) for _ in range(dm.layers))
        self.ln_f = nn.LayerNorm(d)
        self.opt_type_emb = nn.Embedding(dm.n_opt_types, 16)
        self.opt_card = nn.Linear(dc, 64)
        self.opt_attack = nn.Linear(da, 64)
        q_in = 16 + 2 * d + 64 + 64 + dm.opt_f
        self.q_mlp = nn.Sequential(nn.Linear(q_in, d), nn.GELU(), nn.Linear(d, d))
        self.score_mlp = nn.Sequential(nn.Linear(3 * d + G + 64, 256), nn.GELU(), nn.Linear(256, 1))
        nn.init.orthogonal_(self.score_mlp[-1].weight, gain=0.01)
        self.value_mlp = nn.Sequential(nn.Linear(d + G, 256), nn.GELU(), nn.Linear(256, 1))
        if dm.critic == 1:
            if dm.oracle_f != 2 * N_HAND + 3 * N_SPLIT + 2 * N_PRIZE:
                raise ValueError(f"oracle critic needs a {2 * N_HAND + 3 * N_SPLIT + 2 * N_PRIZE}-float oracle block")
            self.oracle_proj = nn.Linear(dc + 6, d)
            self.critic_readout = nn.Parameter(torch.randn(d) * 0.02)
            self.critic_blocks = nn.ModuleList([Block(d, dm.heads, dm.ffn)])
            self.oracle_value_mlp = nn.Sequential(nn.Linear(d + G, 256), nn.GELU(), nn.Linear(256, 1))
            self.aux_hand = nn.Linear(d + G, dm.n_cards)
            self.aux_prize = nn.Linear(d, 1)

    # ---- static tables (pt_static_upload, ptcg_model2.cu:383-419)
    def set_static(self, st):
        """st: dict of numpy arrays card_static (n_cards, 58), att_static
        (n_attacks, 15), card_text (n_cards, 128), att_text (n_attacks, 64),
        skill_text (n_skills, 64), card_attacks (n_cards, 4) and card_skills
        (n_cards, 2) integer ids (0 = empty slot)."""
        dt = next(self.parameters()).dtype
        self.static = {k: torch.as_tensor(v).to(dt) if k in STATIC_SHAPES else torch.as_tensor(v).long()
                       for k, v in st.items()}
        return self

    def tables(self):
        """(card_vec (n_cards, d_c), attack_vec (n_attacks, d_a))."""
        if self.dm.tables == 0:
            return self.card_table, self.attack_table
        if self.static is None:
            raise RuntimeError("static tables not set (set_static)")
        st = self.static
        att = self.attack_mlp(torch.cat([self.attack_id_emb.weight, st["att_static"], st["att_text"]], -1))
        sk = self.skill_mlp(torch.cat([self.skill_id_emb.weight, st["skill_text"]], -1))

        def pools(tab, ids):
            m = (ids > 0).unsqueeze(-1).to(tab.dtype)
            v = tab[ids] * m                      # masked slots are 0-valued participants
            mean = v.sum(1) / m.sum(1).clamp(min=1)
            return mean, first_max_pool(v)

        a_mean, a_max = pools(att, st["card_attacks"])
        s_mean, s_max = pools(sk, st["card_skills"])
        cv = self.card_mlp(torch.cat([self.card_id_emb.weight, st["card_static"], st["card_text"],
                                      a_mean, a_max, s_mean, s_max], -1))
        return cv, att

    # ---- blob IO (native_weights.py:94-113)
    def named_blob_params(self):
        params = dict(self.named_parameters())
        return [(name, params[name]) for name, _ in blob_order(self.dm)]

    def load_blob(self, packed):
        packed = torch.as_tensor(packed, dtype=torch.float32).reshape(-1)
        p = 0
        with torch.no_grad():
            for name, t in self.named_blob_params():
                n = t.numel()
                t.copy_(packed[p:p + n].view_as(t))
                p += n
        if p != packed.numel():
            raise ValueError(f"blob has {packed.numel()} floats, consumed {p}")

    def to_blob(self):
        return torch.cat([t.detach().reshape(-1).float()
                          for _, t in self.named_blob_params()]).numpy()

    def grad_blob(self):
        return torch.cat([(t.grad if t.grad is not None else torch.zeros_like(t))
                          .detach().reshape(-1).float()
                          for _, t in self.named_blob_params()]).numpy()

    # ---- forward
    def _take(self, obs, name):
        a, b = self.off[name]
        return obs[:, a:b]

    def forward(self, obs, return_parts=False):
        dm = self.dm
        B = obs.shape[0]
        L = dm.l_tok
        cv, av = self.tables()
        tok = self._take(obs, "tok_int").reshape(B, L, dm.tok_int)
        ti = tok.long()
        tok_f = self._take(obs, "tok_float").reshape(B, L, dm.tok_f)
        cid = ti[:, :, 0].clamp(0, dm.n_cards - 1)
        t0, t1 = ti[:, :, 3], ti[:, :, 4]
        tool = (cv[t0.clamp(0, dm.n_cards - 1)] * (t0 > 0).unsqueeze(-1).to(cv.dtype)
                + cv[t1.clamp(0, dm.n_cards - 1)] * (t1 > 0).unsqueeze(-1).to(cv.dtype))
        x = self.token_proj(torch.cat([
            cv[cid], tool, tok_f,
            self.zone_emb(ti[:, :, 1].clamp(0, dm.n_zones - 1)),
            self.owner_emb(ti[:, :, 2].clamp(0, dm.n_owners - 1))], dim=-1))

        g = self.global_mlp(self._take(obs, "global_f"))
        di = self._take(obs, "dec_int").long()
        C = lambda i: cv[di[:, i].clamp(0, dm.n_cards - 1)]
        A = lambda i: av[di[:, i].clamp(0, dm.n_attacks - 1)]
        d_vec = self.dec_mlp(torch.cat([
            self.sel_type_emb(di[:, 0].clamp(0, dm.n_select_types - 1)),
            self.ctx_emb(di[:, 1].clamp(0, dm.n_contexts - 1)),
            C(2), C(3), A(4), A(5), C(6), C(7),
            self._take(obs, "dec_float")], dim=-1))
        bc = self.bcast(torch.cat([g, d_vec], dim=-1))

        keep = torch.cat([torch.ones(B, 1, dtype=torch.bool),
                          tok[:, :, 1] > 0], dim=1)
        x = torch.cat([self.readout.expand(B, 1, -1), x + bc.unsqueeze(1)], dim=1)
        for blk in self.blocks:
            x = blk(x, keep)
        h = self.ln_f(x)
        r = h[:, 0]

        NO = dm.n_opt
        oi = self._take(obs, "opt_int").reshape(B, NO, dm.opt_int).long()
        opt_f = self._take(obs, "opt_float").reshape(B, NO, dm.opt_f)

        def ptr(p):
            ok = ((p > 0) & (p <= L)).unsqueeze(-1).to(h.dtype)
            idx = p.clamp(0, L).unsqueeze(-1).expand(-1, -1, dm.d)
            return h.gather(1, idx) * ok

        q = self.q_mlp(torch.cat([
            self.opt_type_emb(oi[:, :, 0].clamp(0, dm.n_opt_types - 1)),
            ptr(oi[:, :, 1]), ptr(oi[:, :, 2]),
            self.opt_card(cv[oi[:, :, 3].clamp(0, dm.n_cards - 1)]),
            self.opt_attack(av[oi[:, :, 4].clamp(0, dm.n_attacks - 1)]),
            opt_f], dim=-1))
        rr = r.unsqueeze(1).expand(-1, NO, -1)
        gg = g.unsqueeze(1).expand(-1, NO, -1)
        dd = d_vec.unsqueeze(1).expand(-1, NO, -1)
        scores = self.score_mlp(torch.cat([q, rr, gg, dd, q * rr], dim=-1)).squeeze(-1)
        rg = torch.cat([r, g], dim=-1)
        blind_v = self.value_mlp(rg)
        parts = dict(h=h, r=r, g=g, d_vec=d_vec, keep=keep, q=q, x0_bc=bc, card_vec=cv, attack_vec=av,
                     blind_v=blind_v)
        if dm.critic == 1:
            value = self._oracle_value(obs, cv, h, keep, g)
            parts["hand_lin"] = self.aux_hand(rg)
            parts["prize_logit"] = self.aux_prize(h[:, 1:]).squeeze(-1)
        else:
            value = blind_v
        out = torch.cat([scores, value], dim=-1)
        if return_parts:
            return out, parts
        return out

    def _oracle_ids(self, obs):
        o = self._take(obs, "oracle")
        H, S, P = N_HAND, N_SPLIT, N_PRIZE
        hand = o[:, :2 * H].reshape(-1, H, 2)
        split = o[:, 2 * H:2 * H + 3 * S].reshape(-1, S, 3)
        prize = o[:, 2 * H + 3 * S:].reshape(-1, P, 2)
        return hand, split, prize

    def _oracle_value(self, obs, cv, h, keep, g):
        """Critic top (model.py:278-308; k_otok_in / k_xc, ptcg_model.cu:441-496)."""
        dm = self.dm
        B = obs.shape[0]
        hand, split, prize = self._oracle_ids(obs)
        H, S, P = N_HAND, N_SPLIT, N_PRIZE
        ids = torch.cat([hand[:, :, 0], split[:, :, 0], prize[:, :, 0]], 1).long()
        feats = torch.zeros(B, H + S + P, 6, dtype=h.dtype)
        feats[:, :H, 0] = 1.0
        feats[:, :H, 3] = hand[:, :, 1]
        feats[:, H:H + S, 1] = 1.0
        feats[:, H:H + S, 4] = split[:, :, 1]
        feats[:, H:H + S, 5] = split[:, :, 2]
        feats[:, H + S:, 2] = 1.0
        feats[:, H + S:, 3] = prize[:, :, 1]
        otok = self.oracle_proj(torch.cat([cv[ids.clamp(0, dm.n_cards - 1)], feats], -1))
        x = torch.cat([self.critic_readout.expand(B, 1, -1), h, otok], 1)
        kc = torch.cat([torch.ones(B, 1, dtype=torch.bool), keep, ids > 0], 1)
        for blk in self.critic_blocks:
            x = blk(x, kc)
        return self.oracle_value_mlp(torch.cat([x[:, 0], g], -1))

    def aux_loss(self, obs, parts, returns):
        """The belief / blind-value losses the native backward applies
        (k_aux_targets, k_hand_grad, k_prize_count/grad, k_blind_grad,
        ptcg_model2.cu:219-285): their autograd gradient is the injected one."""
        dm = self.dm
        B = obs.shape[0]
        NC = dm.n_cards
        dt = parts["h"].dtype
        hand, _, prize = self._oracle_ids(obs)
        # opp-hand count targets: += 4*count at id, ids in (0, NC) except the unknown id NC-1
        hid = hand[:, :, 0].long()
        hcnt = hand[:, :, 1].to(dt) * 4.0
        ok = (hid > 0) & (hid < NC) & (hid != NC - 1) & (hcnt != 0)
        tgt = torch.zeros(B, NC, dtype=dt)
        rows = torch.arange(B).unsqueeze(1).expand_as(hid)
        tgt.index_put_((rows[ok], hid[ok]), hcnt[ok], accumulate=True)
        # my-prize indicator
        pid = prize[:, :, 0].long()
        pok = (pid > 0) & (pid < NC) & (prize[:, :, 1] > 0)
        prized = torch.zeros(B, NC, dtype=dt)
        prows = torch.arange(B).unsqueeze(1).expand_as(pid)
        prized[prows[pok], pid[pok]] = 1.0
        l_hand = AUX_HAND_COEF * ((F.softplus(parts["hand_lin"]) - tgt) ** 2).sum() / (B * NC)
        ret = torch.as_tensor(returns).to(dt).reshape(B, 1)
        l_blind = AUX_VF_COEF * 0.5 * ((parts["blind_v"] - ret) ** 2).sum() / B
        ti = self._take(obs, "tok_int").reshape(B, dm.l_tok, dm.tok_int).long()
        unseen = ti[:, :, 1] == ZONE_MY_UNSEEN
        cnt = max(int(unseen.sum()), 1)
        t = prized.gather(1, ti[:, :, 0].clamp(0, NC - 1))
        bce = F.binary_cross_entropy_with_logits(parts["prize_logit"], t, reduction="none")
        l_prize = AUX_PRIZE_COEF * (bce * unseen.to(dt)).sum() / cnt
        return l_blind + l_hand + l_prize


def build(dm, blob=None, seed=0, dtype=torch.float32, static=None):
    """Construct the oracle; with ``blob`` load those weights, else a
    torch-seeded default init (native_weights.py:116-121 analogue).  The
    static-table model takes its static features in ``static``."""
    torch.manual_seed(seed)
    m = OraclePolicy(dm)
    if blob is not None:
        m.load_blob(blob)
    m = m.to(dtype)
    if static is not None:
        m.set_static(static)
    return m
