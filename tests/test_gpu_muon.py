"""Muon (the reference's optimizer) on the GPU against the oracle
(oracle/muon.py): the alpha / beta GEMM epilogue its Newton-Schulz steps
use, three optimizer steps over the CORE and frozen parameter arenas, the
gate, the trainer with optimizer "muon" against the oracle's minibatch
steps, and the reference's PTCGSTA1 state file.

Tolerances: GEMM epilogue 1e-5 against float64; weights after Muon steps at
relative L2 1e-4 of the update, momentum 1e-5 (the Newton-Schulz products run
in fp32 on the GPU, float64 in the oracle); a closed gate bit-exact.
"""
import ctypes
import struct

import numpy as np
import pytest
import torch

from conftest import rel_l2
from ptcg_amd import dims, native, synth, trainer
import oracle.model as om
import oracle.muon as omu
import oracle.step as ostep

pytestmark = pytest.mark.gpu

P = lambda t: t.data_ptr()


def dev(a, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device="cuda", dtype=dt)


AXPBY_CASES = [(64, 64, 512, 0, 0), (256, 256, 256, 0, 1), (128, 768, 128, 1, 1), (100, 300, 100, 0, 1),
               (1, 1, 256, 0, 0), (33, 130, 33, 1, 1)]


@pytest.mark.parametrize("case", AXPBY_CASES, ids=lambda c: "M%d_N%d_K%d_at%d_bt%d" % c)
def test_gemm_axpby(case, cuda):
    M, N, K, a_t, b_t = case
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(K, M, generator=g) if a_t else torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g) if b_t else torch.randn(N, K, generator=g)
    R = torch.randn(M, N, generator=g)
    alpha, beta = 1.7, -0.6
    opA = A.double().T if a_t else A.double()
    opB = B.double() if b_t else B.double().T
    want = alpha * (opA @ opB) + beta * R.double()
    dA, dB, dR, dC = dev(A), dev(B), dev(R), torch.empty(M, N, device="cuda")
    native.check(native.lib().ptcg_kernel_gemm_axpby(M, N, K, P(dA), A.shape[1], a_t, P(dB), B.shape[1], b_t, P(dC),
                                                     N, alpha, P(dR), N, beta, None))
    torch.cuda.synchronize()
    err = (dC.cpu().double() - want).abs().max() / max(1.0, float(want.abs().max()))
    assert err < 1e-5


class ArenaMuon:
    """The library's Muon over device arenas built from packed blobs."""

    def __init__(self, dm, lr, momentum, wd_1d):
        self.L = native.lib()
        self.dm = dm
        self.cd = dm.as_ctypes()
        self.n = self.L.ptcg_arena_floats(ctypes.byref(self.cd))
        self.packed = self.L.ptcg_packed_floats(ctypes.byref(self.cd))
        h = ctypes.c_void_p()
        native.check(self.L.ptcg_muon_create(ctypes.byref(self.cd), lr, momentum, 0.0, wd_1d, ctypes.byref(h)))
        self.h = h

    def to_arena(self, packed):
        img = np.zeros(self.n, np.float32)
        native.check(self.L.ptcg_packed_to_arena(ctypes.byref(self.cd), np.ascontiguousarray(packed, np.float32)
                                                 .ctypes.data_as(native.c_float_p), img.ctypes.data_as(native.c_float_p)))
        return dev(img)

    def to_packed(self, arena):
        img = arena.cpu().numpy()
        out = np.zeros(self.packed, np.float32)
        native.check(self.L.ptcg_arena_to_packed(ctypes.byref(self.cd), img.ctypes.data_as(native.c_float_p),
                                                 out.ctypes.data_as(native.c_float_p)))
        return out

    def momentum(self):
        """The momentum arena, packed (copied out through a [1, n] -> [n, 1] transpose)."""
        ptr = self.L.ptcg_muon_momentum(self.h)
        t = torch.empty(self.n, device="cuda")
        native.check(self.L.ptcg_transpose_102(P(t), ptr, 1, self.n, 1, 0, None))
        torch.cuda.synchronize()
        return self.to_packed(t)

    def close(self):
        self.L.ptcg_muon_free(self.h)


@pytest.mark.parametrize("dm", [dims.CORE, dims.FROZEN], ids=["core", "frozen"])
def test_muon_steps_match_oracle(dm, cuda):
    ref = om.build(dm, seed=61)
    params = [p for _, p in ref.named_blob_params()]
    w0 = ref.to_blob()
    lr, mu, wd1, max_norm = 0.02, 0.95, 0.01, 0.5
    mu_gpu = ArenaMuon(dm, lr, mu, wd1)
    try:
        W = mu_gpu.to_arena(w0)
        norm = torch.zeros(1, device="cuda")
        opt = omu.OracleMuon(params, lr=lr, momentum=mu, wd_1d=wd1)
        g = torch.Generator().manual_seed(62)
        for it in range(3):
            grads = [torch.randn(p.shape, generator=g) * (0.02 if it != 1 else 2.0) for p in params]   # step 1 clips
            for p, gr in zip(params, grads):
                p.grad = gr
            gpk = torch.cat([gr.reshape(-1) for gr in grads]).numpy()
            G = mu_gpu.to_arena(gpk)
            native.check(mu_gpu.L.ptcg_muon_step(mu_gpu.h, P(W), P(G), max_norm, None, P(norm), None))
            want_norm = opt.step(max_norm)
            torch.cuda.synchronize()
            assert abs(norm.item() - want_norm) <= 1e-5 * want_norm
        w_gpu = mu_gpu.to_packed(W)
        w_ref = ref.to_blob()
        assert rel_l2(w_gpu - w0, w_ref - w0) < 1e-4
        m_ref = torch.cat([m.reshape(-1) for m in opt.mom]).numpy()
        assert rel_l2(mu_gpu.momentum(), m_ref) < 1e-5
    finally:
        mu_gpu.close()


def test_muon_gate_zero_is_noop(cuda):
    dm = dims.tiny()
    ref = om.build(dm, seed=63)
    w0 = ref.to_blob()
    mg = ArenaMuon(dm, 0.02, 0.9, 0.0)
    try:
        W = mg.to_arena(w0)
        G = mg.to_arena(np.full(w0.size, np.nan, np.float32))
        gate = torch.zeros(1, device="cuda")
        native.check(mg.L.ptcg_muon_step(mg.h, P(W), P(G), 0.5, P(gate), None, None))
        torch.cuda.synchronize()
        assert np.array_equal(mg.to_packed(W).view(np.uint32), w0.view(np.uint32))
        assert np.all(mg.momentum() == 0)
    finally:
        mg.close()


HYP = dict(clip_coef=0.2, vf_clip_coef=0.2, vf_coef=0.5, ent_coef=0.01, max_grad_norm=0.5)


def test_trainer_with_muon_matches_oracle(tmp_path, cuda):
    dm, B, steps = dims.tiny(), 32, 3
    lr, mu, wd1 = 0.01, 0.95, 0.05
    ref = om.build(dm, seed=64)
    w0 = ref.to_blob()
    rows = synth.make_obs(dm, 4 * B, seed=65, rich=True)
    inp = synth.make_ppo_inputs(dm, rows, seed=66)
    lists = synth.minibatch_indices(4 * B, B, steps, seed=67, epochs=1)
    pl = trainer.create_pufferl({"dims": dm, "init_weights": w0,
                                 "train": dict(minibatch_size=B, learning_rate=lr, beta1=mu, optimizer="muon",
                                               muon_wd_1d=wd1, **HYP)})
    try:
        trainer.set_rollout(pl, rows, **inp)
        trainer.train(pl, index_lists=lists)
        w_gpu = pl.get_weights()
        pl.global_step, pl.epoch = 1234, 7
        path = tmp_path / "state.bin"
        trainer.save_state(pl, path)
    finally:
        pl.close()
    opt = omu.OracleMuon([p for _, p in ref.named_blob_params()], lr=lr, momentum=mu, wd_1d=wd1)
    ostep.run_update(ref, opt, rows, inp, lists, dict(HYP))
    w_ref = ref.to_blob()
    assert rel_l2(w_gpu - w0, w_ref - w0) < 1e-3
    # PTCGSTA1: magic, int64 global_step, int64 epoch, int64 n, packed weights, packed momentum
    raw = path.read_bytes()
    n = w0.size
    assert raw[:8] == b"PTCGSTA1" and struct.unpack("<qqq", raw[8:32]) == (1234, 7, n)
    assert len(raw) == 32 + 8 * n
    w_file = np.frombuffer(raw[32:32 + 4 * n], np.float32)
    assert np.array_equal(w_file, w_gpu)
    m_file = np.frombuffer(raw[32 + 4 * n:], np.float32)
    m_ref = torch.cat([m.reshape(-1) for m in opt.mom]).numpy()
    assert rel_l2(m_file, m_ref) < 1e-3
    # a fresh Muon trainer resumes from the file
    pl2 = trainer.create_pufferl({"dims": dm, "train": dict(minibatch_size=B, learning_rate=lr, beta1=mu,
                                                            optimizer="muon", **HYP)})
    try:
        trainer.load_state(pl2, path)
        assert np.array_equal(pl2.get_weights(), w_gpu)
        assert (pl2.global_step, pl2.epoch) == (1234, 7)
    finally:
        pl2.close()
