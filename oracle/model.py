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
(ptcg_model.cu:512-517).  Implemented variant: learned card/attack tables
and the blind value head (``value_mlp([r || g])``, model.py:317-318) — the
synthetic workload's model.  The static-table chain and the oracle critic
(model.py:185-205, 278-308) are not restated yet.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .layout import offsets, blob_order


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


class OraclePolicy(nn.Module):
    def __init__(self, dm):
        super().__init__()
        if dm.tables != 0 or dm.critic != 0:
            raise NotImplementedError(
                "oracle restates the learned-table / blind-critic model only")
        self.dm = dm
        d, dc, da, G = dm.d, dm.d_c, dm.d_a, dm.g
        self.off, self.obs_size = offsets(dm)
        self.card_table = nn.Parameter(torch.randn(dm.n_cards, dc))
        self.attack_table = nn.Parameter(torch.randn(dm.n_attacks, da))
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
        cv, av = self.card_table, self.attack_table
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
        value = self.value_mlp(torch.cat([r, g], dim=-1))
        out = torch.cat([scores, value], dim=-1)
        if return_parts:
            return out, dict(h=h, r=r, g=g, d_vec=d_vec, keep=keep, q=q, x0_bc=bc)
        return out


def build(dm, blob=None, seed=0, dtype=torch.float32):
    """Construct the oracle; with ``blob`` load those weights, else a
    torch-seeded default init (native_weights.py:116-121 analogue)."""
    torch.manual_seed(seed)
    m = OraclePolicy(dm)
    if blob is not None:
        m.load_blob(blob)
    return m.to(dtype)
