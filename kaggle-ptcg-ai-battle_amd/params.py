"""Weight-blob layout, arena layout and initial weights.

Blob = packed fp32, tensors in canonical order, no gaps (the reference's
on-disk format, native/tools/native_weights.py:94-113).  Arena = the same
tensors with every tensor start rounded up to a multiple of 4 floats (16 B),
the rule of ``alloc_create`` (native/src/kernels.cu:433-466) that
``packed_blob_to_arena_host`` mirrors (native/src/pufferlib.cu:2366-2390).
The grads arena and the Adam moment arenas share the params arena layout, so
one flat walk with one offset covers all four.
"""
import numpy as np

from .dims import TABLES_LEARNED, TABLES_STATIC, CRITIC_ORACLE

# fixed hidden widths of the reference model (ptcg/rl/model.py:118-175)
OPT_E = 64       # opt_card / opt_attack output
TYPE_E = 16      # opt_type_emb
SC_H = 256       # score_mlp hidden
VAL_H = 256      # value_mlp / oracle_value_mlp hidden
DEC_H = 64       # dec_mlp width
CARD_H = 256     # card_mlp hidden (static tables)
ATT_IN = 127     # 48 id + 15 static + 64 text  (ptcg_model.cu:42)
SK_IN = 112      # 48 id + 64 text              (ptcg_model.cu:43)
CARD_STATIC, CARD_TEXT = 58, 128   # static feature widths (ptcg/rl/cards.py)


def _block(prefix, d, ffn):
    return [
        (f"{prefix}.ln1.weight", (d,)), (f"{prefix}.ln1.bias", (d,)),
        (f"{prefix}.qkv.weight", (3 * d, d)), (f"{prefix}.qkv.bias", (3 * d,)),
        (f"{prefix}.proj.weight", (d, d)), (f"{prefix}.proj.bias", (d,)),
        (f"{prefix}.ln2.weight", (d,)), (f"{prefix}.ln2.bias", (d,)),
        (f"{prefix}.ffn.0.weight", (ffn, d)), (f"{prefix}.ffn.0.bias", (ffn,)),
        (f"{prefix}.ffn.2.weight", (d, ffn)), (f"{prefix}.ffn.2.bias", (d,)),
    ]


def card_in_width(dims):
    """CardVec MLP input (ptcg_model.cu:53): [id64 | static | text | attack
    mean/max | skill mean/max] = 634 at d_a 64 / d_c 128."""
    return 64 + CARD_STATIC + CARD_TEXT + 2 * dims.d_a + 2 * dims.d_c


def param_order(dims):
    """(torch_name, shape) in canonical blob order.

    Static tables + oracle critic reproduce the reference list name for name
    (native/tools/native_weights.py:45-92, PT_PARAMS ptcg_model.cu:95-126).
    Learned tables replace the 13 static-chain tensors with two learned
    tables, ``card_table`` (n_cards, d_c) and ``attack_table``
    (n_attacks, d_a), at the head of the list; the blind critic drops the
    oracle-critic and aux tensors from the tail.  Everything between keeps
    the reference order.
    """
    d, dc, da, G = dims.d, dims.d_c, dims.d_a, dims.g
    card_in = card_in_width(dims)
    if dims.tables == TABLES_STATIC:
        order = [
            ("card_id_emb.weight", (dims.n_cards, 64)),
            ("attack_id_emb.weight", (dims.n_attacks, 48)),
            ("skill_id_emb.weight", (dims.n_skills, 48)),
            ("attack_mlp.0.weight", (da, ATT_IN)), ("attack_mlp.0.bias", (da,)),
            ("skill_mlp.0.weight", (dc, SK_IN)), ("skill_mlp.0.bias", (dc,)),
            ("card_mlp.0.weight", (card_in,)), ("card_mlp.0.bias", (card_in,)),
            ("card_mlp.1.weight", (CARD_H, card_in)), ("card_mlp.1.bias", (CARD_H,)),
            ("card_mlp.3.weight", (dc, CARD_H)), ("card_mlp.3.bias", (dc,)),
        ]
    elif dims.tables == TABLES_LEARNED:
        order = [
            ("card_table", (dims.n_cards, dc)),
            ("attack_table", (dims.n_attacks, da)),
        ]
    else:
        raise ValueError(f"unknown tables mode {dims.tables}")
    order += [
        ("zone_emb.weight", (dims.n_zones, 8)),
        ("owner_emb.weight", (dims.n_owners, 4)),
        ("token_proj.weight", (d, dims.tok_in)), ("token_proj.bias", (d,)),
        ("readout", (d,)),
        ("global_mlp.0.weight", (G, dims.global_f)), ("global_mlp.0.bias", (G,)),
        ("global_mlp.2.weight", (G, G)), ("global_mlp.2.bias", (G,)),
        ("sel_type_emb.weight", (dims.n_select_types, 8)),
        ("ctx_emb.weight", (dims.n_contexts, 32)),
        ("dec_mlp.0.weight", (DEC_H, dims.dec_in)), ("dec_mlp.0.bias", (DEC_H,)),
        ("dec_mlp.2.weight", (DEC_H, DEC_H)), ("dec_mlp.2.bias", (DEC_H,)),
        ("bcast.weight", (d, dims.bcast_in)), ("bcast.bias", (d,)),
    ]
    for i in range(dims.layers):
        order += _block(f"blocks.{i}", d, dims.ffn)
    order += [
        ("ln_f.weight", (d,)), ("ln_f.bias", (d,)),
        ("opt_type_emb.weight", (dims.n_opt_types, TYPE_E)),
        ("opt_card.weight", (OPT_E, dc)), ("opt_card.bias", (OPT_E,)),
        ("opt_attack.weight", (OPT_E, da)), ("opt_attack.bias", (OPT_E,)),
        ("q_mlp.0.weight", (d, dims.q_in)), ("q_mlp.0.bias", (d,)),
        ("q_mlp.2.weight", (d, d)), ("q_mlp.2.bias", (d,)),
        ("score_mlp.0.weight", (SC_H, dims.score_in)), ("score_mlp.0.bias", (SC_H,)),
        ("score_mlp.2.weight", (1, SC_H)), ("score_mlp.2.bias", (1,)),
        ("value_mlp.0.weight", (VAL_H, dims.val_in)), ("value_mlp.0.bias", (VAL_H,)),
        ("value_mlp.2.weight", (1, VAL_H)), ("value_mlp.2.bias", (1,)),
    ]
    if dims.critic == CRITIC_ORACLE:
        order += [
            ("oracle_proj.weight", (d, dc + 6)), ("oracle_proj.bias", (d,)),
            ("critic_readout", (d,)),
        ]
        order += _block("critic_blocks.0", d, dims.ffn)
        order += [
            ("oracle_value_mlp.0.weight", (VAL_H, dims.val_in)),
            ("oracle_value_mlp.0.bias", (VAL_H,)),
            ("oracle_value_mlp.2.weight", (1, VAL_H)),
            ("oracle_value_mlp.2.bias", (1,)),
            ("aux_hand.weight", (dims.n_cards, dims.val_in)),
            ("aux_hand.bias", (dims.n_cards,)),
            ("aux_prize.weight", (1, d)), ("aux_prize.bias", (1,)),
        ]
    return order


def numel(shape):
    n = 1
    for s in shape:
        n *= s
    return n


def packed_size(dims):
    return sum(numel(s) for _, s in param_order(dims))


def arena_offsets(dims):
    """Float offset of each tensor inside the 16 B-aligned arena, and the
    arena size in floats (kernels.cu:433-466: ``offset = (offset+15)&~15``
    in bytes before each tensor).  The size is rounded up to a 16 B multiple
    as well, so flat 128-bit passes over the arena need no tail case."""
    offs, off = [], 0
    for _, shape in param_order(dims):
        off = (off + 3) & ~3
        offs.append(off)
        off += numel(shape)
    return offs, (off + 3) & ~3


def packed_to_arena(dims, packed):
    """pufferlib.cu:2366-2378: scatter a packed blob into an arena image;
    gap floats are zero."""
    packed = np.asarray(packed, dtype=np.float32).ravel()
    want = packed_size(dims)
    if packed.size != want:
        raise ValueError(f"blob has {packed.size} floats, expected {want}")
    offs, total = arena_offsets(dims)
    arena = np.zeros(total, dtype=np.float32)
    p = 0
    for (_, shape), o in zip(param_order(dims), offs):
        n = numel(shape)
        arena[o:o + n] = packed[p:p + n]
        p += n
    return arena


def arena_to_packed(dims, arena):
    """pufferlib.cu:2380-2390: gather the packed blob back out of an arena."""
    arena = np.asarray(arena, dtype=np.float32).ravel()
    offs, total = arena_offsets(dims)
    if arena.size != total:
        raise ValueError(f"arena has {arena.size} floats, expected {total}")
    out = np.empty(packed_size(dims), dtype=np.float32)
    p = 0
    for (_, shape), o in zip(param_order(dims), offs):
        n = numel(shape)
        out[p:p + n] = arena[o:o + n]
        p += n
    return out


def blob_to_dict(dims, packed):
    """name -> ndarray view of a packed blob (native_weights.py:104-113)."""
    packed = np.asarray(packed, dtype=np.float32).ravel()
    out, p = {}, 0
    for name, shape in param_order(dims):
        n = numel(shape)
        out[name] = packed[p:p + n].reshape(shape)
        p += n
    if p != packed.size:
        raise ValueError(f"blob has {packed.size} floats, consumed {p}")
    return out


def dict_to_blob(dims, tensors):
    """native_weights.py:94-101: concatenate tensors in canonical order."""
    chunks = []
    for name, shape in param_order(dims):
        t = np.asarray(tensors[name], dtype=np.float32)
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name}: {t.shape} != {shape}")
        chunks.append(np.ascontiguousarray(t).ravel())
    return np.concatenate(chunks)


def init_blob(dims, seed):
    """Initial weights drawn from the distributions torch's default module
    init uses (nn.Linear: U(+-1/sqrt(fan_in)) for weight and bias;
    nn.Embedding and learned tables: N(0,1); LayerNorm: 1/0; readout
    vectors: N(0, 0.02^2); score head output: orthogonal, gain 0.01 —
    ptcg/rl/model.py:114-175).  Values come from numpy's PCG64, not torch's
    generator, so this blob is NOT bit-identical to a torch-seeded model;
    parity tests load the oracle's blob instead."""
    rng = np.random.Generator(np.random.PCG64(seed))
    out = {}
    order = param_order(dims)
    shapes = dict(order)
    for name, shape in order:
        if name.endswith(".bias"):
            wshape = shapes[name[:-len(".bias")] + ".weight"]
            if len(wshape) == 1:     # LayerNorm bias
                out[name] = np.zeros(shape, np.float32)
                continue
            b = 1.0 / np.sqrt(wshape[1])
            out[name] = rng.uniform(-b, b, shape).astype(np.float32)
        elif name in ("readout", "critic_readout"):
            out[name] = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        elif len(shape) == 1:        # LayerNorm weight
            out[name] = np.ones(shape, np.float32)
        elif name.endswith("emb.weight") or name in ("card_table", "attack_table"):
            out[name] = rng.standard_normal(shape).astype(np.float32)
        elif name == "score_mlp.2.weight":
            v = rng.standard_normal(shape[1])
            out[name] = (0.01 * v / np.linalg.norm(v)).reshape(shape).astype(np.float32)
        else:
            b = 1.0 / np.sqrt(shape[1])
            out[name] = rng.uniform(-b, b, shape).astype(np.float32)
    return dict_to_blob(dims, out)
