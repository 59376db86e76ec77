"""Obs-row layout, weight-blob order and arena rules (CPU).

Pinned against the reference's own numbers: docs/model.md's offsets table
(OBS_SIZE 10944 and each section start), SEAT_COL / FROZEN_COL
(ptcg/rl/buffers.py:233-237, docs/model.md), and the 4 465 812-float /
120-tensor blob (docs/model.md:190-191, native_weights.py:45-92).
"""
import ctypes
import os
import re

import numpy as np
import pytest

from ptcg_amd import dims, params, native
import oracle.layout as ol

FROZEN_OFFSETS = {   # docs/model.md "The observation row" table
    "tok_int": 0, "tok_float": 800, "opt_int": 9760, "opt_float": 10144,
    "opt_mask": 10656, "global_f": 10720, "dec_int": 10784, "dec_float": 10792,
    "oracle": 10808,
}

CONFIGS = [dims.FROZEN, dims.CORE, dims.tiny(), dims.tiny(l_tok=7, n_opt=5, heads=4), dims.tiny_frozen(),
           dims.tiny_frozen(d_c=8, d_a=4)]


def test_frozen_obs_offsets_match_reference_table():
    off, size = dims.build_offsets(dims.FROZEN)
    assert size == 10944
    assert {k: v[0] for k, v in off.items()} == FROZEN_OFFSETS
    # GlobF.ACTOR_SEAT = 31, GlobF.FROZEN_ACTOR = 54 (buffers.py:154,182)
    assert off["global_f"][0] + 31 == 10751
    assert off["global_f"][0] + 54 == 10774


def test_core_obs_size():
    assert dims.CORE.obs_size == 4736


def test_frozen_blob_matches_reference_count():
    order = params.param_order(dims.FROZEN)
    assert len(order) == 120
    assert params.packed_size(dims.FROZEN) == 4465812
    # first / last tensors and the trunk block pattern of native_weights.py
    assert order[0] == ("card_id_emb.weight", (1284, 64))
    assert order[-1] == ("aux_prize.bias", (1,))
    assert ("token_proj.weight", (256, 324)) in order
    assert ("q_mlp.0.weight", (256, 16 + 2 * 256 + 2 * 64 + 8)) in order
    assert ("score_mlp.0.weight", (256, 3 * 256 + 128 + 64)) in order


@pytest.mark.parametrize("dm", CONFIGS, ids=lambda d: f"L{d.l_tok}d{d.d}t{d.tables}c{d.critic}")
def test_oracle_and_package_layouts_agree(dm):
    assert ol.offsets(dm) == dims.build_offsets(dm)
    assert ol.blob_order(dm) == [(n, tuple(s)) for n, s in params.param_order(dm)]


@pytest.mark.parametrize("dm", CONFIGS, ids=lambda d: f"L{d.l_tok}d{d.d}t{d.tables}c{d.critic}")
def test_c_abi_layout_agrees(dm):
    L = native.lib()
    cd = dm.as_ctypes()
    order = params.param_order(dm)
    assert L.ptcg_obs_size(ctypes.byref(cd)) == dm.obs_size
    assert L.ptcg_num_params(ctypes.byref(cd)) == len(order)
    assert L.ptcg_packed_floats(ctypes.byref(cd)) == params.packed_size(dm)
    assert L.ptcg_arena_floats(ctypes.byref(cd)) == params.arena_offsets(dm)[1]
    for i, (name, shape) in enumerate(order):
        nm = ctypes.c_char_p()
        r, c = ctypes.c_int64(), ctypes.c_int64()
        native.check(L.ptcg_param_info(ctypes.byref(cd), i, ctypes.byref(nm), ctypes.byref(r), ctypes.byref(c)))
        assert nm.value.decode() == name
        assert (r.value,) + ((c.value,) if c.value else ()) == tuple(shape)


def test_arena_rule_and_round_trip():
    dm = dims.tiny()
    offs, total = params.arena_offsets(dm)
    assert all(o % 4 == 0 for o in offs) and total % 4 == 0
    rng = np.random.default_rng(0)
    blob = rng.standard_normal(params.packed_size(dm)).astype(np.float32)
    arena = params.packed_to_arena(dm, blob)
    assert np.array_equal(params.arena_to_packed(dm, arena), blob)
    # gap floats are zero and every tensor sits at its aligned offset
    mask = np.zeros(total, bool)
    p = 0
    for (name, shape), o in zip(params.param_order(dm), offs):
        n = params.numel(shape)
        assert np.array_equal(arena[o:o + n], blob[p:p + n])
        mask[o:o + n] = True
        p += n
    assert not arena[~mask].any()
    # the C ABI host helpers produce the same image
    L = native.lib()
    cd = dm.as_ctypes()
    img = np.full(total, 7.0, np.float32)
    native.check(L.ptcg_packed_to_arena(ctypes.byref(cd), native.fptr(blob), native.fptr(img)))
    assert np.array_equal(img, arena)
    back = np.empty_like(blob)
    native.check(L.ptcg_arena_to_packed(ctypes.byref(cd), native.fptr(arena), native.fptr(back)))
    assert np.array_equal(back, blob)


def test_blob_size_mismatch_raises():
    dm = dims.tiny()
    with pytest.raises(ValueError, match="blob has"):
        params.packed_to_arena(dm, np.zeros(5, np.float32))


def _declared_functions():
    names = set()
    inc = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include")
    for f in os.listdir(inc):
        if f.endswith(".h"):
            txt = open(os.path.join(inc, f)).read()
            txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
            names |= set(re.findall(r"\b(ptcg_[a-z0-9_]+)\s*\(", txt))
    return names


def test_library_exports_every_declared_symbol():
    L = native.lib()
    declared = _declared_functions()
    assert len(declared) > 30
    for name in sorted(declared):
        assert hasattr(L, name), f"{name} declared in include/ but not exported"
    # and the ctypes binding covers exactly the declared surface
    assert set(native.exported_symbols()) == declared


def test_init_blob_shapes_and_distributions():
    dm = dims.CORE
    blob = params.init_blob(dm, 0)
    assert blob.size == params.packed_size(dm) and blob.dtype == np.float32
    t = params.blob_to_dict(dm, blob)
    assert np.all(t["blocks.0.ln1.weight"] == 1) and np.all(t["blocks.0.ln1.bias"] == 0)
    b = 1 / np.sqrt(dm.d)
    assert np.abs(t["blocks.0.qkv.weight"]).max() <= b
    assert abs(np.linalg.norm(t["score_mlp.2.weight"]) - 0.01) < 1e-6
    assert np.array_equal(params.init_blob(dm, 0), blob)
