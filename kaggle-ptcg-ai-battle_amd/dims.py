"""Model and observation-row dimensions for the PTCG token-transformer step.

The reference freezes its sizes at compile time (``PT_D/PT_H/PT_FFN/PT_LAYERS``,
native/model/ptcg_model.cu:14-43) and its obs layout in ptcg/rl/buffers.py:29-55.
Here every size is a runtime field of :class:`PtcgDims`, so one build serves
both the reference's frozen layout (``FROZEN``) and the synthetic workload the
benchmarks run (``CORE``: 96 tokens, 32 token features, 2048 card ids,
d256/H4/FFN1024, learned card/attack tables, blind value head).

Field order of :class:`PtcgDims` is the C struct ``PtcgDims`` in
include/ptcg_amd.h; ``as_ctypes`` packs it.
"""
import ctypes
from dataclasses import dataclass, asdict, replace

# table modes / critic modes (ints cross the C ABI)
TABLES_LEARNED = 0   # card/attack vectors are learned (n_cards, d_c)/(n_attacks, d_a) tables
TABLES_STATIC = 1    # the reference's static-table chain (ptcg_model2.cu:422-485)
CRITIC_BLIND = 0     # value = value_mlp([r || g])           (ptcg/rl/model.py:317-318)
CRITIC_ORACLE = 1    # oracle critic block over [creadout || h || oracle tokens]


@dataclass(frozen=True)
class PtcgDims:
    # obs row (ptcg/rl/buffers.py:29-45)
    l_tok: int = 160
    tok_int: int = 5
    tok_f: int = 56
    n_opt: int = 64
    opt_int: int = 6
    opt_f: int = 8
    global_f: int = 64
    dec_int: int = 8
    dec_f: int = 16
    oracle_f: int = 136
    # model (ptcg/rl/model.py:95-175)
    d: int = 256
    heads: int = 8
    ffn: int = 512
    layers: int = 4
    d_c: int = 128
    d_a: int = 64
    g: int = 128
    # vocabularies (ptcg/rl/buffers.py:47-55, ptcg/rl/cards.py:19)
    n_cards: int = 1284
    n_attacks: int = 1573
    n_skills: int = 448
    n_zones: int = 16
    n_owners: int = 4
    n_opt_types: int = 33
    n_select_types: int = 29
    n_contexts: int = 65
    tables: int = TABLES_STATIC
    critic: int = CRITIC_ORACLE

    # ---- derived widths (ptcg_model.cu:44-71, native_weights.py:27-31)
    @property
    def l_seq(self):
        return self.l_tok + 1

    @property
    def dh(self):
        return self.d // self.heads

    @property
    def tok_in(self):      # [card_vec | tool_vec | tok_f | zone8 | owner4]
        return 2 * self.d_c + self.tok_f + 8 + 4

    @property
    def dec_in(self):      # [sel8 | ctx32 | 2 cv | 2 av | 2 cv | dec_f]
        return 8 + 32 + 2 * self.d_c + 2 * self.d_a + 2 * self.d_c + self.dec_f

    @property
    def bcast_in(self):
        return self.g + 64

    @property
    def q_in(self):        # [type16 | h(p1) | h(p2) | ocard64 | oatt64 | opt_f]
        return 16 + 2 * self.d + 64 + 64 + self.opt_f

    @property
    def score_in(self):    # [q | r | g | dvec | q*r]
        return 3 * self.d + self.g + 64

    @property
    def val_in(self):
        return self.d + self.g

    @property
    def obs_size(self):
        return build_offsets(self)[1]

    def offsets(self):
        return build_offsets(self)[0]

    def seat_col(self):
        """Obs column of the actor-seat global feature (GlobF.ACTOR_SEAT = 31,
        ptcg/rl/buffers.py:154,232) that the negamax advantage reads
        (PT_SEAT_COL_M, native/model/ptcg_model2.cu:288)."""
        if self.global_f <= 31:
            raise ValueError(f"global_f={self.global_f} has no actor-seat column (31)")
        return self.offsets()["global_f"][0] + 31

    def as_dict(self):
        return asdict(self)

    def as_ctypes(self):
        return CPtcgDims(*[getattr(self, f) for f, _ in CPtcgDims._fields_])


class CPtcgDims(ctypes.Structure):
    """Mirror of ``struct PtcgDims`` (include/ptcg_amd.h); all fields int32."""
    _fields_ = [(name, ctypes.c_int) for name in (
        "l_tok", "tok_int", "tok_f", "n_opt", "opt_int", "opt_f", "global_f",
        "dec_int", "dec_f", "oracle_f", "d", "heads", "ffn", "layers", "d_c",
        "d_a", "g", "n_cards", "n_attacks", "n_skills", "n_zones", "n_owners",
        "n_opt_types", "n_select_types", "n_contexts", "tables", "critic")]


def build_offsets(dims):
    """Section offsets of one obs row, same recipe as ``_build_offsets``
    (ptcg/rl/buffers.py:212-227): sections laid out back to back in a fixed
    order; returns ({name: (start, end)}, total)."""
    off, cur = {}, 0
    for name, size in [
        ("tok_int", dims.l_tok * dims.tok_int),
        ("tok_float", dims.l_tok * dims.tok_f),
        ("opt_int", dims.n_opt * dims.opt_int),
        ("opt_float", dims.n_opt * dims.opt_f),
        ("opt_mask", dims.n_opt),
        ("global_f", dims.global_f),
        ("dec_int", dims.dec_int),
        ("dec_float", dims.dec_f),
        ("oracle", dims.oracle_f),
    ]:
        off[name] = (cur, cur + size)
        cur += size
    return off, cur


# The reference's frozen layout and default model (buffers.py VERSION 4,
# native_weights.py:24-26, ptcg_model.cu:22-43).
FROZEN = PtcgDims()

# The reference's other documented trunk size, on the same layout and
# variant: d128 / 4 heads / FFN 256 (ptcg_model.cu:19, "A d128/h4 trunk is
# PT_D 128 / PT_H 4 / PT_FFN 256"; head width 32 at both sizes).
FROZEN_D128 = replace(FROZEN, d=128, heads=4, ffn=256)

# The synthetic workload of the benchmark configs: 96 entity tokens, 32
# numeric features per token, card ids in [0, 2048), d256 / 4 heads /
# FFN 1024 / 4 pre-LN layers, 64 options, blind value head, learned tables.
CORE = replace(FROZEN, l_tok=96, tok_f=32, n_cards=2048, heads=4, ffn=1024,
               tables=TABLES_LEARNED, critic=CRITIC_BLIND)


def tiny(**kw):
    """A small CORE-shaped config for fast parity tests."""
    base = dict(l_tok=24, tok_f=8, n_cards=97, n_attacks=33, d=64, heads=2,
                ffn=128, layers=2, d_c=32, d_a=16, g=32, n_opt=16)
    base.update(kw)
    return replace(CORE, **base)


def tiny_frozen(**kw):
    """A small config of the reference's model variant: static-table chain,
    oracle critic and aux heads (for parity tests)."""
    base = dict(tables=TABLES_STATIC, critic=CRITIC_ORACLE, n_skills=21, heads=2)
    base.update(kw)
    return tiny(**base)
