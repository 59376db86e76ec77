"""The HIP path against the reference's own golden vectors (tests/golden/).

Forward: ``debug_forward`` on the fixture's blob, static tables and rows
against ``PTCGTransformer.forward_train`` (ptcg/rl/model.py:326-341): legal
option logits and the oracle-critic value (the (N, 65) output contract,
ptcg_model.cu:512-517).

Backward, through the model's Encoder entry points (ptcg_model_forward /
ptcg_model_backward, ptcg_model4.cu:269-281): the native backward adds the aux
losses' gradients (blind value, hand counts, prizes; ptcg_model4.cu:26-61) to
the gradient of the decoder output.  Two forward + backward calls on the same
rows and weights — decoder gradient G, then decoder gradient 0 — differ by exactly the gradient
of sum(G * out), which the fixture stores for G = its weights on the legal
logits and the oracle value ("C" summaries).  The blind-value aux term is
made ~0 by binding returns equal to the reference's blind value.

Tolerances (fp32 on both sides): logits / value relative L2 <= 1e-5, max|d|
<= 1e-4 * max(1, max|ref|); gradient summaries within 1e-4 of each tensor's
norm; tensors the decoder gradient does not reach (value / aux heads) within
1e-5 of the aux gradient's norm.
"""
import ctypes
import dataclasses

import numpy as np
import pytest
import torch

from conftest import rel_l2
from refvec import load
from ptcg_amd import params, trainer
from ptcg_amd.native import lib, check, fptr

pytestmark = pytest.mark.gpu


class Model:
    """The Encoder entry points of one model on device arenas (torch memory)."""

    def __init__(self, fx, B):
        L = lib()
        self.dm, self.B = fx.dm, B
        self.cd = fx.dm.as_ctypes()
        self.h = ctypes.c_void_p()
        check(L.ptcg_model_create(ctypes.byref(self.cd), ctypes.byref(self.h)))
        n = L.ptcg_arena_floats(ctypes.byref(self.cd))
        img = np.zeros(n, np.float32)
        check(L.ptcg_packed_to_arena(ctypes.byref(self.cd), fptr(np.ascontiguousarray(fx.blob)), fptr(img)))
        self.P = torch.from_numpy(img).cuda()
        self.G = torch.zeros(n, dtype=torch.float32, device="cuda")
        check(L.ptcg_model_bind(self.h, ctypes.c_void_p(self.P.data_ptr()), ctypes.c_void_p(self.G.data_ptr())))
        st = fx.static
        f = [np.ascontiguousarray(st[k], np.float32) for k in
             ("card_static", "att_static", "card_text", "att_text", "skill_text")]
        i = [np.ascontiguousarray(st[k], np.int32) for k in ("card_attacks", "card_skills")]
        check(L.ptcg_model_set_static(self.h, *[a.ctypes.data for a in f + i]))
        check(L.ptcg_model_reg_train(self.h, B))

    def forward(self, obs):
        self.obs = torch.from_numpy(np.ascontiguousarray(obs)).cuda()
        out = ctypes.c_void_p()
        check(lib().ptcg_model_forward(self.h, ctypes.c_void_p(self.obs.data_ptr()), None, self.B,
                                       ctypes.byref(out), None))
        torch.cuda.synchronize()
        return out.value

    def backward(self, grad, returns):
        g = torch.from_numpy(np.ascontiguousarray(grad, np.float32)).cuda()
        self.ret = torch.from_numpy(np.ascontiguousarray(returns, np.float32)).cuda()
        check(lib().ptcg_model_bind_returns(self.h, ctypes.c_void_p(self.ret.data_ptr())))
        check(lib().ptcg_model_backward(self.h, ctypes.c_void_p(g.data_ptr()), None))
        torch.cuda.synchronize()
        img = self.G.cpu().numpy()
        packed = np.empty(params.packed_size(self.dm), np.float32)
        check(lib().ptcg_arena_to_packed(ctypes.byref(self.cd), fptr(img), fptr(packed)))
        return params.blob_to_dict(self.dm, packed)

    def close(self):
        torch.cuda.synchronize()
        lib().ptcg_model_free(self.h)


# The second fixture runs a 4-head trunk (head width 64, FFN 1024, 2 layers)
# on the frozen layout's 161-position trunk and 218-position critic.
GPU_CASES = ("frozen", "h4ffn1024")


@pytest.fixture(scope="module", params=GPU_CASES)
def fx(request):
    return load(request.param)


def test_unsupported_attention_shape_is_rejected(cuda):
    """A head width the fused attention kernels do not take (128) is refused
    at creation with a clear message."""
    f = load("h4ffn1024")
    dm = dataclasses.replace(f.dm, heads=f.dm.d // 128)
    with pytest.raises(RuntimeError, match="attention shape"):
        trainer.create_pufferl({"dims": dm, "static": f.static, "train": dict(minibatch_size=f.obs.shape[0])})


def _check_forward(fx, out):
    z = fx.z
    legal = fx.legal()
    A = fx.dm.n_opt
    for got, want in ((out[:, :A][legal], z["logits"][legal]), (out[:, A:], z["oracle_v"])):
        scale = max(1.0, float(np.abs(want).max()))
        assert rel_l2(got, want) <= 1e-5, rel_l2(got, want)
        assert np.abs(got - want).max() <= 1e-4 * scale


def test_debug_forward_matches_reference(fx, cuda):
    B = fx.obs.shape[0]
    pl = trainer.create_pufferl({"dims": fx.dm, "init_weights": fx.blob, "static": fx.static,
                                 "train": dict(minibatch_size=B)})
    out = trainer.debug_forward(pl, fx.obs)
    _check_forward(fx, out)
    pl.close()


def test_model_backward_matches_reference(fx, cuda):
    from conftest import d2h
    B = fx.obs.shape[0]
    A = fx.dm.n_opt
    m = Model(fx, B)
    out_ptr = m.forward(fx.obs)
    _check_forward(fx, d2h(out_ptr, (B, A + 1)))
    z = fx.z
    G = np.zeros((B, A + 1), np.float32)
    G[:, :A] = np.where(fx.legal(), z["w_logits"], 0.0)
    G[:, A] = z["w_oracle_v"][:, 0]
    returns = z["blind_v"][:, 0]
    g_full = {k: v.copy() for k, v in m.backward(G, returns).items()}
    m.forward(fx.obs)   # the backward may reuse activation memory: forward again
    g_aux = m.backward(np.zeros_like(G), returns)
    m.close()
    diff = {k: g_full[k].astype(np.float64) - g_aux[k] for k in g_full}
    norms = z["gC_norm"]
    reached = [n for i, n in enumerate(fx.names) if norms[i] > 0]
    unreached = [n for i, n in enumerate(fx.names) if norms[i] == 0]
    bad = fx.grad_check("C", {n: diff[n] if n in reached else np.zeros_like(diff[n]) for n in fx.names})
    assert not bad, bad[:8]
    for n in unreached:   # the value and aux heads get the aux gradient only
        lim = 1e-5 * max(float(np.linalg.norm(g_aux[n])), 1e-3)
        assert float(np.linalg.norm(diff[n])) <= lim, n
    assert {"aux_hand.weight", "aux_prize.weight", "value_mlp.0.weight"} <= set(unreached)
