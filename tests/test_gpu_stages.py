"""Stage dumps for parity bisection (the reference's PTCG_DUMP_DIR,
native/model/ptcg_model3.cu:371-400): with the variable set, a forward writes
every named stage as raw fp32 in the full (sample, position) layout.  The
dumped stages equal the oracle's intermediates on the same rows and weights
(relative L2 <= 1e-5), in the compact-trunk layout (CORE-shaped model) and
the full-length one (the reference variant); rows the compact trunk did not
compute read 0."""
import os

import numpy as np
import pytest
import torch

from conftest import rel_l2
from ptcg_amd import dims, synth, trainer
import oracle.model as om

pytestmark = pytest.mark.gpu

STAGES = ("card_vec", "att_tab", "tok_cat", "tokp", "dec_in", "g_out", "d_out", "bc_out", "keep", "h", "q_in",
          "q_vec", "sc_in", "out")


@pytest.mark.parametrize("dm", [dims.tiny(), dims.tiny_frozen()], ids=["compact", "variant"])
def test_stage_dump_matches_oracle(dm, tmp_path, cuda):
    B = 6
    st = synth.make_static(dm, 7) if dm.tables == 1 else None
    ref = om.build(dm, seed=5, static=st)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": ref.to_blob(), "static": st,
                                 "train": dict(minibatch_size=B)})
    obs = synth.make_obs(dm, B, seed=6, rich=True)
    os.environ["PTCG_DUMP_DIR"] = str(tmp_path)
    try:
        out = trainer.debug_forward(pl, obs)
    finally:
        del os.environ["PTCG_DUMP_DIR"]
    pl.close()
    want, parts = ref(torch.from_numpy(obs), return_parts=True)
    P = {k: (v.detach().double().numpy() if torch.is_tensor(v) else v) for k, v in parts.items()}
    ld = lambda n: np.fromfile(tmp_path / f"{n}.bin", np.float32)
    for n in STAGES + ("x0",) + tuple(f"x{i}" for i in range(1, dm.layers + 1)):
        assert (tmp_path / f"{n}.bin").exists(), n
    Ls, D = dm.l_tok + 1, dm.d
    assert rel_l2(ld("out").reshape(B, -1), want.detach().numpy()) < 1e-5
    assert np.array_equal(ld("out").reshape(B, -1), out)
    assert rel_l2(ld("card_vec").reshape(P["card_vec"].shape), P["card_vec"]) < 1e-5
    assert rel_l2(ld("att_tab").reshape(P["attack_vec"].shape), P["attack_vec"]) < 1e-5
    assert rel_l2(ld("g_out").reshape(B, -1), P["g"]) < 1e-5
    assert rel_l2(ld("d_out").reshape(B, -1), P["d_vec"]) < 1e-5
    assert rel_l2(ld("bc_out").reshape(B, -1), P["x0_bc"]) < 1e-5
    keep = P["keep"].astype(bool)
    assert np.array_equal(ld("keep").reshape(B, Ls) != 0, keep)
    h = ld("h").reshape(B, Ls, D)
    assert rel_l2(h[keep], P["h"][keep]) < 1e-5
    q = ld("q_vec").reshape(B, dm.n_opt, D)
    assert rel_l2(q, P["q"]) < 1e-5
    assert ld("tok_cat").size == B * dm.l_tok * (2 * dm.d_c + dm.tok_f + 12)
    assert ld("tokp").size == B * dm.l_tok * D
    if dm.critic == 0:
        # the compact trunk computes READOUT, the valid tokens and the
        # pointer targets; a padded position no pointer names reads 0
        x0 = ld("x0").reshape(B, Ls, D)
        oi = obs[:, slice(*dm.offsets()["opt_int"])].reshape(B, dm.n_opt, dm.opt_int)
        named = np.zeros((B, Ls), bool)
        for n in range(B):
            for p in oi[n, :, 1:3].astype(int).ravel():
                if 0 < p <= dm.l_tok:
                    named[n, p] = True
        idle = ~keep & ~named
        assert idle.any() and not np.any(x0[idle])
