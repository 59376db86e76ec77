"""Run-to-run determinism of the training backward on the GPU.

The reference adds the embedding-table gradients with fp32 atomics
(native/model/ptcg_model2.cu k_*_bwd), so its sums change with the order the
adds land in.  Here every reduction has a fixed order and the table scatters
add in 64-bit fixed point, so two identical forward + backward calls give
bit-identical gradient arenas, and the index-list path (rows gathered by
index) gives the same bits as the same rows passed contiguously.  Checked on
the learned-table model and on the static-table variant (pool backward,
CardVec rows shared by tokens / options / oracle tokens), at a batch where
many rows share padding ids and hot option types.
"""
import numpy as np
import pytest

from conftest import rel_l2
from ptcg_amd import dims, params, synth, trainer
import oracle.model as om

pytestmark = pytest.mark.gpu

HYP = dict(clip_coef=0.2, vf_clip_coef=0.2, vf_coef=0.5, ent_coef=0.01, max_grad_norm=0.5)


def _make(dm, B, seed, static, precision="fp32"):
    st = synth.make_static(dm, seed + 1000) if static else None
    ref = om.build(dm, seed=seed, static=st)
    cfg = {"dims": dm, "init_weights": ref.to_blob(), "precision": precision,
           "train": dict(minibatch_size=B, **HYP)}
    if static:
        cfg["static"] = st
    return trainer.create_pufferl(cfg)


CASES = [(dims.tiny(), 32, False, "fp32"), (dims.CORE, 64, False, "fp32"), (dims.tiny_frozen(), 24, True, "fp32"),
         (dims.FROZEN, 8, True, "fp32"), (dims.CORE, 64, False, "bf16"), (dims.tiny_frozen(), 24, True, "bf16")]


@pytest.mark.parametrize("dm,B,static,precision", CASES,
                         ids=["tiny", "core", "tiny_frozen", "frozen", "core_bf16", "tiny_frozen_bf16"])
def test_backward_bitwise_repeatable(dm, B, static, precision, cuda):
    """fp32, and the bf16 variant (bf16 activations, split-K weight gradients
    with fixed-order sums, the same fixed-point table sums)."""
    pl = _make(dm, B, seed=71, static=static, precision=precision)
    try:
        R = 3 * B
        rows = synth.make_obs(dm, R, seed=72, rich=True)
        inp = synth.make_ppo_inputs(dm, rows, seed=73)
        idx = np.random.default_rng(74).choice(R, B, replace=False).astype(np.int32)
        d_rows = pl.to_device(rows)
        d_all = {k: pl.to_device(v) for k, v in inp.items()}
        grads = []
        for _ in range(2):
            pl.forward_backward(d_rows, pl.to_device(idx, np.int32), d_all)
            pl.sync()
            grads.append(pl.get_grads())
        g = params.blob_to_dict(dm, grads[0])
        tables = [k for k in g if "emb" in k or "tab" in k]
        assert tables and any(np.any(g[k]) for k in tables)
        assert np.array_equal(grads[0], grads[1]), rel_l2(grads[1], grads[0])
        # the same rows passed contiguously
        sel = {k: pl.to_device(v[idx]) for k, v in inp.items()}
        pl.forward_backward(pl.to_device(rows[idx]), None, sel)
        pl.sync()
        g_cont = pl.get_grads()
        assert np.array_equal(grads[0], g_cont), rel_l2(g_cont, grads[0])
    finally:
        pl.close()
