"""Obs-row offsets and weight-blob order, restated for the oracle.

Independent of the product package on purpose: tests compare the two, and
both against the reference's frozen numbers.

* offsets: ptcg/rl/buffers.py:212-230 (``_build_offsets``).
* blob order: native/tools/native_weights.py:34-92 (``param_order``), with
  the learned-table / blind-critic variant used by the synthetic workload.
"""

SECTIONS = ("tok_int", "tok_float", "opt_int", "opt_float", "opt_mask",
            "global_f", "dec_int", "dec_float", "oracle")


def offsets(dm):
    """buffers.py:212-227 — sections back to back in fixed order."""
    sizes = {
        "tok_int": dm.l_tok * dm.tok_int,
        "tok_float": dm.l_tok * dm.tok_f,
        "opt_int": dm.n_opt * dm.opt_int,
        "opt_float": dm.n_opt * dm.opt_f,
        "opt_mask": dm.n_opt,
        "global_f": dm.global_f,
        "dec_int": dm.dec_int,
        "dec_float": dm.dec_f,
        "oracle": dm.oracle_f,
    }
    off, cur = {}, 0
    for name in SECTIONS:
        off[name] = (cur, cur + sizes[name])
        cur += sizes[name]
    return off, cur


def blob_order(dm):
    """native_weights.py:34-92 — (name, shape) in blob order."""
    d, ffn = dm.d, dm.ffn
    tok_in = 2 * dm.d_c + dm.tok_f + 8 + 4
    dec_in = 8 + 32 + 2 * dm.d_c + 2 * dm.d_a + 2 * dm.d_c + dm.dec_f
    q_in = 16 + 2 * d + 2 * 64 + dm.opt_f
    score_in = 3 * d + dm.g + 64
    val_in = d + dm.g
    card_in = 64 + 58 + 128 + 2 * dm.d_a + 2 * dm.d_c   # 634 at d_a 64 / d_c 128

    def block(p):
        return [(f"{p}.ln1.weight", (d,)), (f"{p}.ln1.bias", (d,)),
                (f"{p}.qkv.weight", (3 * d, d)), (f"{p}.qkv.bias", (3 * d,)),
                (f"{p}.proj.weight", (d, d)), (f"{p}.proj.bias", (d,)),
                (f"{p}.ln2.weight", (d,)), (f"{p}.ln2.bias", (d,)),
                (f"{p}.ffn.0.weight", (ffn, d)), (f"{p}.ffn.0.bias", (ffn,)),
                (f"{p}.ffn.2.weight", (d, ffn)), (f"{p}.ffn.2.bias", (d,))]

    if dm.tables == 1:     # static-table chain (native_weights.py:48-55)
        order = [("card_id_emb.weight", (dm.n_cards, 64)),
                 ("attack_id_emb.weight", (dm.n_attacks, 48)),
                 ("skill_id_emb.weight", (dm.n_skills, 48)),
                 ("attack_mlp.0.weight", (dm.d_a, 127)), ("attack_mlp.0.bias", (dm.d_a,)),
                 ("skill_mlp.0.weight", (dm.d_c, 112)), ("skill_mlp.0.bias", (dm.d_c,)),
                 ("card_mlp.0.weight", (card_in,)), ("card_mlp.0.bias", (card_in,)),
                 ("card_mlp.1.weight", (256, card_in)), ("card_mlp.1.bias", (256,)),
                 ("card_mlp.3.weight", (dm.d_c, 256)), ("card_mlp.3.bias", (dm.d_c,))]
    else:
        order = [("card_table", (dm.n_cards, dm.d_c)),
                 ("attack_table", (dm.n_attacks, dm.d_a))]
    order += [("zone_emb.weight", (dm.n_zones, 8)), ("owner_emb.weight", (dm.n_owners, 4)),
              ("token_proj.weight", (d, tok_in)), ("token_proj.bias", (d,)),
              ("readout", (d,)),
              ("global_mlp.0.weight", (dm.g, dm.global_f)), ("global_mlp.0.bias", (dm.g,)),
              ("global_mlp.2.weight", (dm.g, dm.g)), ("global_mlp.2.bias", (dm.g,)),
              ("sel_type_emb.weight", (dm.n_select_types, 8)),
              ("ctx_emb.weight", (dm.n_contexts, 32)),
              ("dec_mlp.0.weight", (64, dec_in)), ("dec_mlp.0.bias", (64,)),
              ("dec_mlp.2.weight", (64, 64)), ("dec_mlp.2.bias", (64,)),
              ("bcast.weight", (d, dm.g + 64)), ("bcast.bias", (d,))]
    for i in range(dm.layers):
        order += block(f"blocks.{i}")
    order += [("ln_f.weight", (d,)), ("ln_f.bias", (d,)),
              ("opt_type_emb.weight", (dm.n_opt_types, 16)),
              ("opt_card.weight", (64, dm.d_c)), ("opt_card.bias", (64,)),
              ("opt_attack.weight", (64, dm.d_a)), ("opt_attack.bias", (64,)),
              ("q_mlp.0.weight", (d, q_in)), ("q_mlp.0.bias", (d,)),
              ("q_mlp.2.weight", (d, d)), ("q_mlp.2.bias", (d,)),
              ("score_mlp.0.weight", (256, score_in)), ("score_mlp.0.bias", (256,)),
              ("score_mlp.2.weight", (1, 256)), ("score_mlp.2.bias", (1,)),
              ("value_mlp.0.weight", (256, val_in)), ("value_mlp.0.bias", (256,)),
              ("value_mlp.2.weight", (1, 256)), ("value_mlp.2.bias", (1,))]
    if dm.critic == 1:     # oracle critic + aux heads (native_weights.py:81-90)
        order += [("oracle_proj.weight", (d, dm.d_c + 6)), ("oracle_proj.bias", (d,)),
                  ("critic_readout", (d,))]
        order += block("critic_blocks.0")
        order += [("oracle_value_mlp.0.weight", (256, val_in)),
                  ("oracle_value_mlp.0.bias", (256,)),
                  ("oracle_value_mlp.2.weight", (1, 256)),
                  ("oracle_value_mlp.2.bias", (1,)),
                  ("aux_hand.weight", (dm.n_cards, val_in)), ("aux_hand.bias", (dm.n_cards,)),
                  ("aux_prize.weight", (1, d)), ("aux_prize.bias", (1,))]
    return order
