"""The allocation-free PPO loss entry point (ptcg_ppo_loss_fwd_bwd_noalloc)
against the allocating one (ptcg_ppo_loss_fwd_bwd), through the C ABI.

Both run the same kernels in the same order, so every output (gradient,
ratio, new value, the seven statistics + count, the guard pair) is compared
bit for bit.  Calls in a row share the library's scratch array: a large call,
then a smaller one (whose partials overwrite only a prefix of the first
call's), then the maximum row count; one row more is rejected on the host.
"""
import numpy as np
import pytest
import torch

from ptcg_amd import native

pytestmark = pytest.mark.gpu

MAX_ROWS = 65536   # PT_PPO_NOALLOC_MAX_ROWS in include/ptcg_amd.h


def _inputs(n, A, seed):
    rng = np.random.default_rng(seed)
    scores = rng.standard_normal((n, A + 1)).astype(np.float32)
    mask = (rng.random((n, A)) < 0.4).astype(np.float32)
    mask[np.arange(n), rng.integers(0, A, n)] = 1
    acts = (mask.cumsum(1) >= 1).argmax(1).astype(np.float32)   # first legal option
    old = rng.normal(-2, 0.5, n).astype(np.float32)
    adv = rng.standard_normal(n).astype(np.float32)
    ret = rng.standard_normal(n).astype(np.float32)
    val = (ret - adv + rng.normal(0, 0.3, n)).astype(np.float32)
    idx = rng.permutation(n).astype(np.int32)
    return [torch.from_numpy(a).cuda() for a in (scores, mask, acts, old, adv, ret, val, idx)]


def _run(fn, ins, n, A, ent):
    scores, mask, acts, old, adv, ret, val, idx = ins
    out = [torch.zeros(n * (A + 1), device="cuda"), torch.zeros(n, device="cuda"), torch.zeros(n, device="cuda"),
           torch.zeros(8, device="cuda"), torch.zeros(2, device="cuda")]
    native.check(fn(scores.data_ptr(), n, A, mask.data_ptr(), A, idx.data_ptr(), acts.data_ptr(), old.data_ptr(),
                    adv.data_ptr(), ret.data_ptr(), val.data_ptr(), None, 0.2, 0.2, 0.5, ent.data_ptr(),
                    *[t.data_ptr() for t in out], None))
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in out]


@pytest.mark.parametrize("sizes", [[(4096, 64), (37, 64), (MAX_ROWS, 64)], [(512, 17), (2, 5)]])
def test_noalloc_equals_allocating_entry_point(sizes, cuda):
    L = native.lib()
    ent = torch.tensor([0.01], device="cuda")
    for k, (n, A) in enumerate(sizes):
        print(f"noalloc ppo loss: call {k}, n={n}, A={A}", flush=True)
        ins = _inputs(n, A, 100 + k)
        want = _run(L.ptcg_ppo_loss_fwd_bwd, ins, n, A, ent)
        got = _run(L.ptcg_ppo_loss_fwd_bwd_noalloc, ins, n, A, ent)
        for w, g in zip(want, got):
            assert np.array_equal(w.view(np.uint32), g.view(np.uint32)), (n, A)
        assert got[3][7] == 1.0 and np.any(got[0])


def test_noalloc_rejects_oversized(cuda):
    L = native.lib()
    a = torch.zeros(8, device="cuda")
    p = a.data_ptr()
    with pytest.raises(native.PtcgError, match="scratch"):
        native.check(L.ptcg_ppo_loss_fwd_bwd_noalloc(p, MAX_ROWS + 1, 64, p, 64, None, p, p, p, p, p, None,
                                                     0.2, 0.2, 0.5, p, p, None, None, None, None, None))
