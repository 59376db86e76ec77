"""Kernel-level parity on the GPU, through the C ABI (include/ptcg_amd_kernels.h
and the PPO / Adam entry points of include/ptcg_amd.h).

References: float64 torch on the CPU for GEMM / LayerNorm / attention (the
oracle's attention restatement), the oracle PPO loss and Adam.  Tolerance:
relative L2 error <= 1e-5 and max error <= 1e-4 of the reference's max for
fp32 kernels (written per test).
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from conftest import rel_l2, max_rel
from ptcg_amd import native
import oracle.ppo as oppo
import oracle.adam as oadam

pytestmark = pytest.mark.gpu


def dev(a, dtype=torch.float32):
    return torch.as_tensor(np.ascontiguousarray(a)).to(dtype).to("cuda")


def empty(*shape):
    return torch.zeros(*shape, dtype=torch.float32, device="cuda")


def P(t):
    return None if t is None else t.data_ptr()


def gelu(x):
    return 0.5 * x * (1 + torch.erf(x / math.sqrt(2.0)))


def gelu_grad(x):
    return 0.5 * (1 + torch.erf(x / math.sqrt(2.0))) + x * torch.exp(-0.5 * x * x) / math.sqrt(2 * math.pi)


GEMM_CASES = [
    # M, N, K, a_t, b_t, epi
    (37, 52, 300, 0, 0, 0), (37, 52, 300, 0, 0, 1), (130, 68, 64, 0, 0, 2),
    (256, 256, 256, 0, 0, 3), (200, 96, 40, 0, 1, 4), (64, 300, 256, 0, 1, 0),
    (64, 128, 20000, 1, 1, 0), (768, 256, 4096, 1, 1, 0), (96, 36, 12, 1, 0, 0),
    (129, 132, 132, 0, 1, 5), (512, 1024, 256, 0, 0, 2),
    # widths / leading dimensions that are not multiples of 4 (the reference's
    # 127-wide attack input, 634-wide card input, 134-wide oracle token input)
    (1573, 64, 127, 0, 0, 2), (1284, 634, 256, 0, 1, 0), (300, 256, 134, 0, 0, 1),
    (64, 127, 1573, 1, 1, 0), (45, 33, 17, 1, 0, 5), (256, 634, 20000, 1, 1, 0),
    # more tiles than compute units with a small remainder: the balanced launch
    # (whole tiles + a split-K tail reduced through the epilogue)
    (34000, 256, 256, 0, 0, 2), (33000, 384, 256, 0, 1, 4), (33024, 256, 512, 0, 0, 5),
    (33100, 256, 256, 0, 0, 3),
    # a GELU layer keeping gelu'(z): forward (6) and the multiply backward (7),
    # on the LDS-DMA kernel (K = 172: a last k-tile ending inside the stage) and
    # a balanced launch
    (512, 1024, 256, 0, 0, 6), (300, 256, 172, 0, 0, 6), (34000, 256, 256, 0, 0, 6),
    (512, 1024, 256, 0, 1, 7), (200, 96, 40, 0, 1, 7), (33000, 384, 256, 0, 1, 7),
    # k-contiguous K % 16 != 0 at the model's sizes (option query 664 wide,
    # token concat 300 wide with a balanced tail) and split K ending mid-stage
    (13000, 256, 664, 0, 0, 6), (37000, 256, 300, 0, 0, 1), (64, 64, 4100, 0, 0, 0), (96, 64, 2052, 0, 1, 5),
    # many K splits: partial sums reduced by split groups (accumulate and store)
    (64, 128, 20000, 0, 1, 5), (256, 256, 20000, 1, 1, 0), (200, 260, 9000, 1, 1, 0),
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: "M%d_N%d_K%d_at%d_bt%d_e%d" % c)
def test_gemm_layouts_and_epilogues(case, cuda):
    M, N, K, a_t, b_t, epi = case
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    A = torch.randn(K, M, generator=g) if a_t else torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g) if b_t else torch.randn(N, K, generator=g)
    bias = torch.randn(N, generator=g)
    R = torch.randn(M, N, generator=g)
    C0 = torch.randn(M, N, generator=g)
    Am = (A.T if a_t else A).double()
    Bm = (B if b_t else B.T).double()
    acc = Am @ Bm
    ref2 = None
    if epi == 0: ref = acc
    elif epi == 1: ref = acc + bias.double()
    elif epi == 2:
        ref = acc + bias.double()
        ref2 = gelu(ref)
    elif epi == 3: ref = acc + bias.double() + R.double()
    elif epi == 4: ref = acc * gelu_grad(R.double())
    elif epi == 6:
        z = acc + bias.double()
        ref, ref2 = gelu_grad(z), gelu(z)
    elif epi == 7: ref = acc * R.double()
    else: ref = C0.double() + acc
    dA, dB, dbias, dR = dev(A), dev(B), dev(bias), dev(R)
    dC = dev(C0) if epi == 5 else empty(M, N)
    dC2 = empty(M, N)
    ws = empty(32 << 20)
    L = native.lib()
    native.check(L.ptcg_kernel_gemm(M, N, K, P(dA), M if a_t else K, a_t, P(dB), N if b_t else K, b_t,
                                    P(dC), N, epi, P(dbias), P(dR), N, P(dC2), N, P(ws), ws.numel(), None))
    torch.cuda.synchronize()
    got = dC.cpu().double()
    assert rel_l2(got, ref) < 1e-5 and max_rel(got, ref) < 1e-4, (rel_l2(got, ref), max_rel(got, ref))
    if ref2 is not None:
        got2 = dC2.cpu().double()
        assert rel_l2(got2, ref2) < 1e-5


DEV_ROWS_CASES = [
    # rows computed, N, K, B transposed, epilogue: the sync-free model's 256-wide
    # products (dX: B transposed, STORE / MUL; forward: BIAS / BIAS_RESID /
    # BIAS_GELU_D) with between one and four tiles per CU, K with a partial
    # last k-tile (300), fewer tiles than CUs, more than four per CU
    (37400, 256, 1024, 1, 0), (37400, 256, 768, 1, 7), (33333, 256, 256, 1, 0),
    (40000, 256, 1024, 0, 3), (34567, 256, 300, 0, 1), (36000, 256, 256, 0, 6),
    (900, 256, 256, 1, 0), (70000, 256, 256, 0, 1),
]


@pytest.mark.parametrize("rows,N,K,b_t,epi", DEV_ROWS_CASES)
def test_gemm_device_rows(rows, N, K, b_t, epi, cuda):
    """A launch sized for a row bound that computes the device count's rows
    (the sync-free model's form) against float64; rows past the count keep
    their contents.  With B not transposed it balances its last wave from
    the device count as the host-count launch does (same tiles, K splits and
    partial-sum order): the same bits where the host count runs unsplit (at
    least 512 tiles); otherwise (dX layouts: one pass over K per tile) fp32
    accumulation-order agreement with the host-count launch."""
    bound = rows + 3000
    g = torch.Generator().manual_seed(rows + K + epi)
    A = torch.randn(bound, K, generator=g)
    B = torch.randn(K, N, generator=g) if b_t else torch.randn(N, K, generator=g)
    bias = torch.randn(N, generator=g)
    R = torch.randn(bound, N, generator=g)
    acc = A[:rows].double() @ (B.double() if b_t else B.double().T)
    ref2 = None
    if epi == 0: ref = acc
    elif epi == 1: ref = acc + bias.double()
    elif epi == 3: ref = acc + bias.double() + R[:rows].double()
    elif epi == 6:
        z = acc + bias.double()
        ref, ref2 = gelu_grad(z), gelu(z)
    else: ref = acc * R[:rows].double()
    dA, dB, dbias, dR = dev(A), dev(B), dev(bias), dev(R)
    ldb = N if b_t else K
    ws = empty(32 << 20)
    L = native.lib()
    sentinel = 7.0
    dC, dC2 = torch.full((bound, N), sentinel, device="cuda"), torch.full((bound, N), sentinel, device="cuda")
    rows_dev = torch.tensor([rows], dtype=torch.int32, device="cuda")
    native.check(L.ptcg_kernel_gemm_rows_dev(bound, N, K, P(dA), K, P(dB), ldb, b_t, P(dC), N, epi, P(dbias),
                                             P(dR), N, P(dC2), N, P(rows_dev), P(ws), ws.numel(), None))
    hC, hC2 = empty(rows, N), empty(rows, N)
    native.check(L.ptcg_kernel_gemm(rows, N, K, P(dA), K, 0, P(dB), ldb, b_t, P(hC), N, epi, P(dbias), P(dR), N,
                                    P(hC2), N, P(ws), ws.numel(), None))
    torch.cuda.synchronize()
    got = dC[:rows].cpu().double()
    assert rel_l2(got, ref) < 1e-5 and max_rel(got, ref) < 1e-4, (rel_l2(got, ref), max_rel(got, ref))
    assert bool((dC[rows:] == sentinel).all())
    if ref2 is not None:
        assert rel_l2(dC2[:rows].cpu().double(), ref2) < 1e-5
        assert bool((dC2[rows:] == sentinel).all())
    assert rel_l2(got, hC.cpu().double()) < 5e-6
    if ref2 is not None:
        assert rel_l2(dC2[:rows].cpu().double(), hC2.cpu().double()) < 5e-6
    if not b_t and ((rows + 127) // 128) * ((N + 127) // 128) >= 512:
        assert torch.equal(dC[:rows], hC)
        if ref2 is not None:
            assert torch.equal(dC2[:rows], hC2)


def test_gemm_operand_not_16b_aligned(cuda):
    # aligned widths, but A starts one float into its buffer: scalar-load path
    g = torch.Generator().manual_seed(5)
    A = torch.randn(200 * 64 + 1, generator=g)
    B = torch.randn(96, 64, generator=g)
    dA, dB, dC = dev(A), dev(B), empty(200, 96)
    native.check(native.lib().ptcg_kernel_gemm(200, 96, 64, dA.data_ptr() + 4, 64, 0, P(dB), 64, 0, P(dC), 96, 0,
                                               None, None, 0, None, 0, None, 0, None))
    torch.cuda.synchronize()
    ref = A[1:].view(200, 64).double() @ B.double().T
    assert rel_l2(dC.cpu().double(), ref) < 1e-5


@pytest.mark.parametrize("rows,inp,out", [(6000, 256, 768), (1573, 127, 64), (100, 64, 36), (8192, 1024, 256)])
def test_gemm_weight_grad_with_bias_sums(rows, inp, out, cuda):
    g = torch.Generator().manual_seed(rows + inp)
    dY = torch.randn(rows, out, generator=g)
    X = torch.randn(rows, inp, generator=g)
    d_dY, d_X, dW, db = dev(dY), dev(X), empty(out, inp), empty(out)
    ws = empty(32 << 20)
    native.check(native.lib().ptcg_kernel_gemm_dw(rows, inp, out, P(d_dY), out, P(d_X), inp, P(dW), P(db),
                                                  P(ws), ws.numel(), None))
    torch.cuda.synchronize()
    refW = dY.double().T @ X.double()
    refb = dY.double().sum(0)
    assert rel_l2(dW.cpu().double(), refW) < 1e-5
    assert rel_l2(db.cpu().double(), refb) < 1e-5


# (row bound, device rows, in, out): the sync-free trunk's weight gradients at
# B = 512 (49 664-row bound, 37.4k rows: the bound's split rule gives two
# workgroups per CU, the device count one), a count below 1 024 rows under a
# bound above it (the rule's chunk floor changes there), a small product, and
# no rows at all
@pytest.mark.parametrize("bound,rows,inp,out", [(49664, 37400, 256, 1024), (49664, 37400, 1024, 256),
                                                (49664, 37400, 256, 768), (2000, 900, 256, 256),
                                                (1500, 1100, 64, 36), (49664, 0, 256, 256)])
def test_gemm_weight_grad_device_rows(bound, rows, inp, out, cuda):
    """dW = dY^T X and db = column sums of dY over a device row count below
    the launch's bound: against float64 over those rows, and against the
    host-count launch of the same rows to fp32 accumulation-order accuracy
    (both split the rows by the same rule)."""
    g = torch.Generator().manual_seed(bound + rows + inp)
    dY = torch.randn(bound, out, generator=g)
    X = torch.randn(bound, inp, generator=g)
    d_dY, d_X, dW, db = dev(dY), dev(X), empty(out, inp), empty(out)
    rows_dev = torch.tensor([rows], dtype=torch.int32, device="cuda")
    ws = empty(32 << 20)
    L = native.lib()
    native.check(L.ptcg_kernel_gemm_dw_rows_dev(bound, inp, out, P(d_dY), out, P(d_X), inp, P(dW), P(db),
                                                P(rows_dev), P(ws), ws.numel(), None))
    torch.cuda.synchronize()
    if rows == 0:
        assert not bool(dW.any()) and not bool(db.any())
        return
    refW = dY[:rows].double().T @ X[:rows].double()
    refb = dY[:rows].double().sum(0)
    assert rel_l2(dW.cpu().double(), refW) < 1e-5
    assert rel_l2(db.cpu().double(), refb) < 1e-5
    hW, hb = empty(out, inp), empty(out)
    native.check(L.ptcg_kernel_gemm_dw(rows, inp, out, P(d_dY), out, P(d_X), inp, P(hW), P(hb), P(ws), ws.numel(),
                                       None))
    torch.cuda.synchronize()
    assert rel_l2(dW.cpu().double(), hW.cpu().double()) < 5e-6
    assert rel_l2(db.cpu().double(), hb.cpu().double()) < 5e-6


# one launch up to 4 096 rows (1 row, fewer rows than row groups, a tail
# past the four interleaved accumulators), two levels past it
@pytest.mark.parametrize("M,N", [(1000, 300), (1, 70), (13, 64), (4096, 512), (4097, 100), (20000, 300)])
def test_colsum(M, N, cuda):
    X = torch.randn(M, N, generator=torch.Generator().manual_seed(M + N))
    out = empty(N)
    ws = empty(1 << 20)
    dX = dev(X)
    native.check(native.lib().ptcg_kernel_colsum(P(dX), N, M, N, P(out), P(ws), ws.numel(), None))
    torch.cuda.synchronize()
    assert rel_l2(out.cpu(), X.double().sum(0)) < 1e-6


# rows: one row, a partial 64-row tile, whole tiles, the trunk's 37.4k rows;
# bf16: bf16 operands and LayerNorm output (the mixed-precision blocks)
@pytest.mark.parametrize("rows,K,bf16", [(1, 256, 0), (63, 256, 0), (200, 1024, 0), (1024, 256, 0),
                                         (37417, 256, 0), (3001, 1024, 0), (1, 256, 1), (200, 1024, 1),
                                         (37417, 256, 1), (3001, 1024, 1)])
def test_gemm_resid_ln(rows, K, bf16, cuda):
    """The residual product fused with the LayerNorm that reads it: C, y,
    mean and rstd against float64 (C = A W^T + bias + R; y = LN(C) w + b),
    bit-equal to the unfused pair (the plain product, no split, then the
    LayerNorm kernel; bf16: the bf16-operand product, and y rounded to bf16
    by round to nearest even), and a device row count leaves the later rows
    alone."""
    N = 256
    g = torch.Generator().manual_seed(rows + K + bf16)
    A = torch.randn(rows, K, generator=g) / math.sqrt(K)
    W = torch.randn(N, K, generator=g)
    if bf16:   # the products see bf16-rounded operands
        A, W = A.bfloat16().float(), W.bfloat16().float()
    bias = torch.randn(N, generator=g) * 0.1
    R = torch.randn(rows, N, generator=g) * 2 + 0.5
    lw = torch.randn(N, generator=g)
    lb = torch.randn(N, generator=g)
    C64 = A.double() @ W.double().T + bias.double() + R.double()
    y64 = torch.nn.functional.layer_norm(C64, (N,), lw.double(), lb.double(), eps=1e-5)
    mu64 = C64.mean(1)
    rs64 = 1.0 / torch.sqrt(C64.var(1, unbiased=False) + 1e-5)
    L = native.lib()
    ot = torch.bfloat16 if bf16 else torch.float32
    dA, dW = dev(A, ot), dev(W, ot)
    db, dR, dlw, dlb = dev(bias), dev(R), dev(lw), dev(lb)
    C, mu, rs = empty(rows, N), empty(rows), empty(rows)
    y = torch.zeros(rows, N, dtype=ot, device="cuda")
    native.check(L.ptcg_kernel_gemm_resid_ln(rows, K, P(dA), P(dW), P(db), P(dR), P(C), P(dlw), P(dlb), P(y),
                                             P(mu), P(rs), bf16, None, None))
    # the unfused pair: EPI_BIAS_RESID (3) without a workspace (no split-K, no tail), then LayerNorm
    C2, y2, mu2, rs2 = empty(rows, N), empty(rows, N), empty(rows), empty(rows)
    if bf16:
        native.check(L.ptcg_kernel_gemm_bs(rows, N, K, P(dA), K, P(dW), K, P(C2), N, 3, 0, P(db), P(dR), N,
                                           None, 0, None))
    else:
        native.check(L.ptcg_kernel_gemm(rows, N, K, P(dA), K, 0, P(dW), K, 0, P(C2), N, 3, P(db), P(dR), N,
                                        None, 0, None, 0, None))
    native.check(L.ptcg_kernel_layernorm_fwd(P(C2), P(dlw), P(dlb), P(y2), P(mu2), P(rs2), rows, N, None))
    torch.cuda.synchronize()
    assert rel_l2(C.cpu(), C64) < 1e-6 and max_rel(C.cpu(), C64) < 1e-5
    if bf16:   # y rounded to bf16: half an ulp of 2^-8 relative
        assert rel_l2(y.float().cpu(), y64) < 4e-3
    else:
        assert rel_l2(y.cpu(), y64) < 1e-5 and max_rel(y.cpu(), y64) < 1e-4
    assert rel_l2(mu.cpu(), mu64) < 1e-5 and rel_l2(rs.cpu(), rs64) < 1e-5
    for a, b in ((C, C2), (y, y2.to(ot)), (mu, mu2), (rs, rs2)):
        assert torch.equal(a, b)
    if rows > 64:
        # device row count: rows past it keep their contents
        cut = rows // 2 + 5
        nd = torch.tensor([cut], dtype=torch.int32, device="cuda")
        C3 = torch.full((rows, N), 7.0, device="cuda")
        y3 = torch.full((rows, N), 7.0, dtype=ot, device="cuda")
        mu3, rs3 = torch.full((rows,), 7.0, device="cuda"), torch.full((rows,), 7.0, device="cuda")
        native.check(L.ptcg_kernel_gemm_resid_ln(rows, K, P(dA), P(dW), P(db), P(dR), P(C3), P(dlw), P(dlb),
                                                 P(y3), P(mu3), P(rs3), bf16, P(nd), None))
        torch.cuda.synchronize()
        assert torch.equal(C3[:cut], C[:cut]) and torch.equal(y3[:cut], y[:cut])
        assert torch.equal(mu3[:cut], mu[:cut]) and torch.equal(rs3[:cut], rs[:cut])
        assert bool((C3[cut:] == 7.0).all()) and bool((y3[cut:] == 7.0).all())
        assert bool((mu3[cut:] == 7.0).all()) and bool((rs3[cut:] == 7.0).all())


# rows: one row, a partial 64-row tile, whole tiles, the trunk's 37.4k rows;
# K: the FFN1 (1024) and QKV (768) dX products of a bf16 block
@pytest.mark.parametrize("rows,K,res", [(1, 1024, 1), (63, 768, 0), (200, 1024, 1), (1024, 768, 1),
                                        (3001, 1024, 0), (37417, 1024, 1), (37417, 768, 1)])
def test_gemm_dx_layernorm_bwd(rows, K, res, cuda):
    """The bf16 dX product fused with the LayerNorm backward that reads it:
    dx, dw, db against float64 (dy = dY WT^T; dx = rs (g - mean g - xh
    mean(g xh)) + dres with g = dy w, xh = (x - mu) rs; dw = sum dy xh, db =
    sum dy), against the unfused pair (the bf16 product, then the LayerNorm
    backward kernel), the bf16 copy of dx rounded to nearest even, and a
    device row count that leaves the later rows alone and sums dw / db over
    the rows before it."""
    N = 256
    g = torch.Generator().manual_seed(rows + K + res)
    dY = (torch.randn(rows, K, generator=g) / math.sqrt(K)).bfloat16().float()
    WT = torch.randn(N, K, generator=g).bfloat16().float()
    x = torch.randn(rows, N, generator=g) * 1.5 + 0.3
    w = torch.randn(N, generator=g)
    mu = x.double().mean(1)
    rs = 1.0 / torch.sqrt(x.double().var(1, unbiased=False) + 1e-5)
    mu, rs = mu.float(), rs.float()
    dres = torch.randn(rows, N, generator=g) if res else None

    def ref(n):
        dy = dY[:n].double() @ WT.double().T
        xh = (x[:n].double() - mu[:n, None].double()) * rs[:n, None].double()
        gg = dy * w.double()
        dx = rs[:n, None].double() * (gg - gg.mean(1, keepdim=True) - xh * (gg * xh).mean(1, keepdim=True))
        if res:
            dx = dx + dres[:n].double()
        return dy, dx, (dy * xh).sum(0), dy.sum(0)

    dy64, dx64, dw64, db64 = ref(rows)
    L = native.lib()
    d_dY, d_WT = dev(dY, torch.bfloat16), dev(WT, torch.bfloat16)
    dx_, dw_, dmu, drs = dev(x), dev(w), dev(mu), dev(rs)
    d_dres = dev(dres) if res else None
    ws = empty(1 << 21)
    gx, gxh, gw, gb = empty(rows, N), torch.zeros(rows, N, dtype=torch.bfloat16, device="cuda"), empty(N), empty(N)
    native.check(L.ptcg_kernel_gemm_dx_layernorm_bwd(rows, K, P(d_dY), P(d_WT), P(dx_), P(dw_), P(dmu), P(drs),
                                                     P(d_dres), P(gx), P(gxh), P(gw), P(gb), P(ws), ws.numel(),
                                                     None, None))
    # the unfused pair: the bf16 product (EPI_STORE, no workspace), then the LayerNorm backward
    dy2, gx2, gw2, gb2 = empty(rows, N), empty(rows, N), empty(N), empty(N)
    native.check(L.ptcg_kernel_gemm_bs(rows, N, K, P(d_dY), K, P(d_WT), K, P(dy2), N, 0, 0, None, None, 0,
                                       None, 0, None))
    native.check(L.ptcg_kernel_layernorm_bwd(P(dy2), P(dx_), P(dw_), P(dmu), P(drs), P(d_dres), P(gx2),
                                             P(gw2), P(gb2), rows, N, P(ws), ws.numel(), None))
    torch.cuda.synchronize()
    assert rel_l2(dy2.cpu(), dy64) < 1e-6
    assert rel_l2(gx.cpu(), dx64) < 1e-5 and rel_l2(gx.cpu(), gx2.cpu()) < 1e-6
    assert rel_l2(gw.cpu(), dw64) < 1e-5 and rel_l2(gw.cpu(), gw2.cpu()) < 1e-6
    assert rel_l2(gb.cpu(), db64) < 1e-5 and rel_l2(gb.cpu(), gb2.cpu()) < 1e-6
    assert torch.equal(gxh, gx.bfloat16())
    if rows > 64:
        # device row count: rows past it keep their contents, dw / db cover the rows before it
        cut = rows // 2 + 5
        nd = torch.tensor([cut], dtype=torch.int32, device="cuda")
        gx3 = torch.full((rows, N), 7.0, device="cuda")
        gxh3 = torch.full((rows, N), 7.0, dtype=torch.bfloat16, device="cuda")
        gw3, gb3 = empty(N), empty(N)
        native.check(L.ptcg_kernel_gemm_dx_layernorm_bwd(rows, K, P(d_dY), P(d_WT), P(dx_), P(dw_), P(dmu),
                                                         P(drs), P(d_dres), P(gx3), P(gxh3), P(gw3), P(gb3),
                                                         P(ws), ws.numel(), P(nd), None))
        torch.cuda.synchronize()
        assert torch.equal(gx3[:cut], gx[:cut]) and torch.equal(gxh3[:cut], gxh[:cut])
        assert bool((gx3[cut:] == 7.0).all()) and bool((gxh3[cut:] == 7.0).all())
        _, _, dw_c, db_c = ref(cut)
        assert rel_l2(gw3.cpu(), dw_c) < 1e-5 and rel_l2(gb3.cpu(), db_c) < 1e-5


def test_gemm_dx_layernorm_bwd_rejects_other_shapes(cuda):
    L = native.lib()
    a, wt = torch.zeros(8, 100, dtype=torch.bfloat16, device="cuda"), torch.zeros(256, 100, dtype=torch.bfloat16,
                                                                                  device="cuda")
    x, gx, v, st = empty(8, 256), empty(8, 256), empty(256), empty(8)
    ws = empty(1 << 16)
    with pytest.raises(RuntimeError, match="layernorm bwd"):
        native.check(L.ptcg_kernel_gemm_dx_layernorm_bwd(8, 100, P(a), P(wt), P(x), P(v), P(st), P(st), None,
                                                         P(gx), None, P(v), P(v), P(ws), ws.numel(), None, None))
    # a shape that fits, with a null dY or a null W^T: rejected on the host
    a2, wt2 = torch.zeros(8, 128, dtype=torch.bfloat16, device="cuda"), torch.zeros(256, 128, dtype=torch.bfloat16,
                                                                                    device="cuda")
    for pa, pw in ((None, P(wt2)), (P(a2), None)):
        with pytest.raises(RuntimeError, match="null buffer"):
            native.check(L.ptcg_kernel_gemm_dx_layernorm_bwd(8, 128, pa, pw, P(x), P(v), P(st), P(st), None,
                                                             P(gx), None, P(v), P(v), P(ws), ws.numel(), None, None))


def test_gemm_resid_ln_rejects_other_shapes(cuda):
    L = native.lib()
    a, w, b, r = empty(8, 100), empty(256, 100), empty(256), empty(8, 256)
    out = [empty(8, 256), empty(256), empty(256), empty(8, 256), empty(8), empty(8)]
    with pytest.raises(RuntimeError, match="gemm \\+ layernorm"):
        native.check(L.ptcg_kernel_gemm_resid_ln(8, 100, P(a), P(w), P(b), P(r), P(out[0]), P(out[1]), P(out[2]),
                                                 P(out[3]), P(out[4]), P(out[5]), 0, None, None))


# (20001, 256): several row pairs per wave in the backward and an odd tail;
# (5, 256): fewer rows than one workgroup's waves
@pytest.mark.parametrize("rows,D", [(1000, 256), (37, 64), (130, 1024), (9, 300), (1284, 634), (50, 127),
                                    (20001, 256), (5, 256), (33, 512), (700, 1024)])
def test_layernorm_fwd_bwd(rows, D, cuda):
    g = torch.Generator().manual_seed(rows + D)
    x = (torch.randn(rows, D, generator=g) * 3 + 1).double().requires_grad_()
    w = (torch.randn(D, generator=g)).double().requires_grad_()
    b = (torch.randn(D, generator=g)).double().requires_grad_()
    dy = torch.randn(rows, D, generator=g).double()
    dres = torch.randn(rows, D, generator=g).double()
    y = torch.nn.functional.layer_norm(x, (D,), w, b, eps=1e-5)
    y.backward(dy)
    L = native.lib()
    dx_, dw_, db_ = dev(x.detach()), dev(w.detach()), dev(b.detach())
    yy, mu, rs = empty(rows, D), empty(rows), empty(rows)
    native.check(L.ptcg_kernel_layernorm_fwd(P(dx_), P(dw_), P(db_), P(yy), P(mu), P(rs), rows, D, None))
    gx, gw, gb = empty(rows, D), empty(D), empty(D)
    ws = empty(1 << 20)
    d_dy, d_dres = dev(dy), dev(dres)
    native.check(L.ptcg_kernel_layernorm_bwd(P(d_dy), P(dx_), P(dw_), P(mu), P(rs), P(d_dres), P(gx),
                                             P(gw), P(gb), rows, D, P(ws), ws.numel(), None))
    torch.cuda.synchronize()
    assert rel_l2(yy.cpu(), y.detach()) < 1e-6
    assert rel_l2(gx.cpu(), x.grad + dres) < 1e-5
    assert rel_l2(gw.cpu(), w.grad) < 1e-5
    assert rel_l2(gb.cpu(), b.grad) < 1e-5


def _attn_ref(qkv, keep, H, Dh):
    """Oracle attention (oracle/model.py Block.attention, fp64) on (N,L,3D)."""
    N, L, D3 = qkv.shape
    D = D3 // 3
    q, k, v = qkv.view(N, L, 3, H, Dh).permute(2, 0, 3, 1, 4).unbind(0)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(Dh)
    s = s.masked_fill(~keep[:, None, None, :], -1e30)
    p = torch.softmax(s, -1)
    return (p @ v).transpose(1, 2).reshape(N, L, D), torch.logsumexp(s, -1)


# (N, L, H, Dh, path): path bit 1 = backward with dS in LDS, bit 2 = recompute
ATTN_CASES = [(6, 97, 4, 64, 3), (5, 25, 2, 32, 3), (3, 100, 2, 64, 3), (4, 64, 8, 32, 3), (2, 1, 4, 64, 3),
              (3, 128, 2, 32, 3), (2, 17, 1, 64, 3),
              # rows too long for dS in LDS: the reference's trunk (161) and critic (218) at Dh 32
              (2, 140, 2, 32, 5), (3, 161, 8, 32, 5), (2, 218, 8, 32, 5), (1, 256, 2, 32, 5), (2, 140, 2, 64, 5),
              # head width 64 beyond 144 positions (one split-pair workgroup per CU): the
              # reference variant's trunk and critic with 4 heads, and the longest row
              (3, 161, 4, 64, 5), (2, 218, 4, 64, 5), (1, 256, 2, 64, 5), (2, 150, 1, 64, 5)]


@pytest.mark.parametrize("N,L,H,Dh,path", ATTN_CASES, ids=lambda *a: None)
def test_attention_fwd_bwd(N, L, H, Dh, path, cuda):
    assert native.lib().ptcg_kernel_attention_path(L, Dh) == path
    g = torch.Generator().manual_seed(N * L + H)
    D = H * Dh
    qkv = torch.randn(N, L, 3 * D, generator=g).double().requires_grad_()
    keep = torch.rand(N, L, generator=g) < 0.7
    keep[:, 0] = True
    ctx, lse = _attn_ref(qkv, keep, H, Dh)
    dctx = torch.randn(N, L, D, generator=g).double()
    ctx.backward(dctx)
    L_ = native.lib()
    dq = dev(qkv.detach())
    dk = dev(keep.float())
    c, l = empty(N, L, D), empty(N, H, L)
    native.check(L_.ptcg_kernel_attention_fwd(P(dq), P(dk), P(c), P(l), N, L, H, Dh, None))
    gq = empty(N, L, 3 * D)
    d_dctx = dev(dctx)
    native.check(L_.ptcg_kernel_attention_bwd(P(dq), P(dk), P(c), P(l), P(d_dctx), P(gq), N, L, H, Dh, None))
    torch.cuda.synchronize()
    assert rel_l2(c.cpu(), ctx.detach()) < 1e-5
    assert rel_l2(l.cpu(), lse.detach()) < 1e-6
    assert rel_l2(gq.cpu(), qkv.grad) < 1e-5
    # masked keys receive no gradient in K and V
    gk = gq.cpu().view(N, L, 3, D)
    assert torch.all(gk[:, :, 1:][~keep] == 0)


@pytest.mark.parametrize("N,L,H,Dh,path", ATTN_CASES, ids=lambda *a: None)
def test_attention_bf16_products(N, L, H, Dh, path, cuda):
    """bf16 products (operands rounded to bf16, fp32 softmax and sums)
    against the float64 reference: context, log-sum-exp and dqkv within bf16
    tolerances (8-bit mantissa, ~4e-3 relative per rounded operand), and
    further from it than the fp32 kernels are (the products really are bf16);
    masked keys still receive exactly zero K / V gradient."""
    g = torch.Generator().manual_seed(N * L + H + 7)
    D = H * Dh
    qkv = torch.randn(N, L, 3 * D, generator=g).double().requires_grad_()
    keep = torch.rand(N, L, generator=g) < 0.7
    keep[:, 0] = True
    ctx, lse = _attn_ref(qkv, keep, H, Dh)
    dctx = torch.randn(N, L, D, generator=g).double()
    ctx.backward(dctx)
    L_ = native.lib()
    dq, dk, d_dctx = dev(qkv.detach()), dev(keep.float()), dev(dctx)
    c, l, gq = empty(N, L, D), empty(N, H, L), empty(N, L, 3 * D)
    native.check(L_.ptcg_kernel_attention_fwd_bf16(P(dq), P(dk), P(c), P(l), N, L, H, Dh, None))
    native.check(L_.ptcg_kernel_attention_bwd_bf16(P(dq), P(dk), P(c), P(l), P(d_dctx), P(gq), N, L, H, Dh, None))
    torch.cuda.synchronize()
    e_c, e_l, e_g = rel_l2(c.cpu(), ctx.detach()), rel_l2(l.cpu(), lse.detach()), rel_l2(gq.cpu(), qkv.grad)
    assert e_c < 1e-2 and e_l < 1e-2 and e_g < 3e-2, (e_c, e_l, e_g)
    if L > 1:
        assert e_c > 1e-4 and e_g > 1e-4
    gk = gq.cpu().view(N, L, 3, D)
    assert torch.all(gk[:, :, 1:][~keep] == 0)


@pytest.mark.parametrize("N,L,H,Dh,path", [c for c in ATTN_CASES if c[4] & 2], ids=lambda *a: None)
@pytest.mark.parametrize("bf16", [0, 1])
def test_attention_bwd_global_ds(N, L, H, Dh, path, bf16, cuda):
    """The backward with dS parked in a global scratch (the model's training
    form: LDS holds only Q and dO) against float64 at the same bars as the
    LDS form, and beside that form's own result; the scratch is filled with
    NaN first, so a dS entry read before it is written would show."""
    g = torch.Generator().manual_seed(N * L + H + 11 * bf16)
    D = H * Dh
    qkv = torch.randn(N, L, 3 * D, generator=g).double().requires_grad_()
    keep = torch.rand(N, L, generator=g) < 0.7
    keep[:, 0] = True
    ctx, lse = _attn_ref(qkv, keep, H, Dh)
    dctx = torch.randn(N, L, D, generator=g).double()
    ctx.backward(dctx)
    L_ = native.lib()
    nbytes = L_.ptcg_kernel_attention_bwd_ws_bytes(N, L, H, Dh, bf16)
    lp = 16 * ((L + 15) // 16)
    assert nbytes == N * H * lp * lp * (2 if bf16 else 4)
    ws = torch.full((nbytes // 4,), float("nan"), device="cuda")
    dq, dk, d_dctx = dev(qkv.detach()), dev(keep.float()), dev(dctx)
    c, l, g_lds, g_ws = empty(N, L, D), empty(N, H, L), empty(N, L, 3 * D), empty(N, L, 3 * D)
    fwd = L_.ptcg_kernel_attention_fwd_bf16 if bf16 else L_.ptcg_kernel_attention_fwd
    bwd = L_.ptcg_kernel_attention_bwd_bf16 if bf16 else L_.ptcg_kernel_attention_bwd
    native.check(fwd(P(dq), P(dk), P(c), P(l), N, L, H, Dh, None))
    native.check(bwd(P(dq), P(dk), P(c), P(l), P(d_dctx), P(g_lds), N, L, H, Dh, None))
    native.check(L_.ptcg_kernel_attention_bwd_ws(P(dq), P(dk), P(c), P(l), P(d_dctx), P(g_ws), N, L, H, Dh, bf16,
                                                 P(ws), nbytes, None))
    torch.cuda.synchronize()
    e_ws, e_lds = rel_l2(g_ws.cpu(), qkv.grad), rel_l2(g_lds.cpu(), qkv.grad)
    if bf16:
        assert e_ws < 3e-2, e_ws
        assert rel_l2(g_ws.cpu(), g_lds.cpu()) < 1e-2
    else:
        assert e_ws < 1e-5, (e_ws, e_lds)
        assert rel_l2(g_ws.cpu(), g_lds.cpu()) < 2e-6
    # dK and dV are produced by pass A in both forms: identical bits
    gw, gl = g_ws.cpu().view(N, L, 3, D), g_lds.cpu().view(N, L, 3, D)
    assert torch.equal(gw[:, :, 1:], gl[:, :, 1:])
    assert torch.all(gw[:, :, 1:][~keep] == 0)
    # a scratch one byte short is refused
    with pytest.raises(native.PtcgError, match="workspace"):
        native.check(L_.ptcg_kernel_attention_bwd_ws(P(dq), P(dk), P(c), P(l), P(d_dctx), P(g_ws), N, L, H, Dh,
                                                     bf16, P(ws), nbytes - 1, None))


def test_attention_rejects_oversized(cuda):
    a = empty(4)
    with pytest.raises(native.PtcgError, match="LDS"):
        native.check(native.lib().ptcg_kernel_attention_fwd(P(a), P(a), P(a), P(a), 1, 300, 1, 64, None))
    assert native.lib().ptcg_kernel_attention_path(257, 64) == -1
    assert native.lib().ptcg_kernel_attention_path(257, 32) == -1
    assert native.lib().ptcg_kernel_attention_path(97, 48) == -1


def _ppo_inputs(n, A, seed):
    rng = np.random.default_rng(seed)
    scores = rng.standard_normal((n, A + 1)).astype(np.float32)
    mask = (rng.random((n, A)) < 0.4).astype(np.float32)
    mask[np.arange(n), rng.integers(0, A, n)] = 1
    acts = np.array([rng.choice(np.flatnonzero(m)) for m in mask], np.float32)
    old = rng.normal(-2, 0.5, n).astype(np.float32)
    adv = rng.standard_normal(n).astype(np.float32)
    ret = rng.standard_normal(n).astype(np.float32)
    val = (ret - adv + rng.normal(0, 0.3, n)).astype(np.float32)
    return scores, mask, acts, old, adv, ret, val


@pytest.mark.parametrize("n,A", [(512, 64), (37, 64), (64, 17), (2048, 64)])
def test_ppo_loss_matches_oracle(n, A, cuda):
    scores, mask, acts, old, adv, ret, val = _ppo_inputs(n, A, n + A)
    kw = dict(clip=0.2, vf_clip=0.2, vf_coef=0.5, ent_coef=0.01)
    T = lambda a: torch.from_numpy(a).double()
    ref = oppo.ppo_loss(T(scores), T(mask), T(acts), T(old), T(adv), T(ret), T(val), **kw)
    grad, ratio, nv = empty(n, A + 1), empty(n), empty(n)
    stats, guard = empty(8), empty(2)
    idx = np.random.default_rng(1).permutation(n).astype(np.int32)
    # rows gathered through row_idx: inputs stored permuted
    inv = np.argsort(idx)
    L = native.lib()
    keep = [dev(a) for a in (scores, mask, acts, old, adv, ret, val)]   # hold device buffers
    ent = dev(np.array([0.01], np.float32))   # device scalar, as in a captured step
    native.check(L.ptcg_ppo_loss_fwd_bwd(
        P(keep[0]), n, A, P(keep[1]), A, None, *[P(t) for t in keep[2:]], None,
        0.2, 0.2, 0.5, P(ent), P(grad), P(ratio), P(nv), P(stats), P(guard), None))
    torch.cuda.synchronize()
    assert rel_l2(grad.cpu(), ref["grad"]) < 1e-5
    assert rel_l2(ratio.cpu(), ref["ratio"]) < 1e-6
    st = stats.cpu().double()
    assert np.allclose(st[:7], ref["stats"], rtol=1e-5, atol=1e-6)
    assert st[7] == 1.0
    assert abs(guard[0].item() - ref["stats"][5].item()) < 1e-5 + 1e-5 * abs(ref["stats"][5].item())
    # row_idx path: per-row inputs live at permuted rows
    grad2 = empty(n, A + 1)
    # stored so that row r's data sits at position idx[r]
    keep2 = [dev(a[inv]) for a in (mask, acts, old, adv, ret, val)] + [dev(idx, torch.int32)]
    native.check(L.ptcg_ppo_loss_fwd_bwd(
        P(keep[0]), n, A, P(keep2[0]), A, P(keep2[6]), *[P(t) for t in keep2[1:6]], None,
        0.2, 0.2, 0.5, P(ent), P(grad2), None, None, None, None, None))
    torch.cuda.synchronize()
    assert rel_l2(grad2.cpu(), ref["grad"]) < 1e-5


def test_kl_gate(cuda):
    L = native.lib()
    for kl, vf, kt, vt, want in [(0.01, 0.1, 0.05, 0.5, 1.0), (0.06, 0.1, 0.05, 0.5, 0.0),
                                 (float("nan"), 0.1, 0.05, 0.5, 0.0), (float("nan"), 0.1, 0.0, 0.5, 1.0),
                                 (0.01, float("inf"), 0.05, 0.5, 0.0), (0.01, 0.7, 0.05, 0.0, 1.0)]:
        g, sk = empty(1), empty(2)
        gd = dev(np.array([kl, vf], np.float32))
        native.check(L.ptcg_kl_gate(P(gd), kt, vt, P(g), P(sk), None))
        torch.cuda.synchronize()
        assert g.item() == want == oppo.kl_gate(kl, vf, kt, vt)
        # every veto, then the vetoes whose value test failed (KL test off)
        assert sk[0].item() == 1.0 - want
        assert sk[1].item() == 1.0 - oppo.kl_gate(kl, vf, 0.0, vt)


def lr_dev(lr):
    """Adam's learning rate as the device double the kernel reads."""
    return torch.tensor([lr], dtype=torch.float64, device="cuda")


def _adam_case(n, seed):
    rng = np.random.default_rng(seed)
    p = rng.standard_normal(n).astype(np.float32)
    g = (rng.standard_normal(n) * 0.1).astype(np.float32)
    return p, g


@pytest.mark.parametrize("n,max_norm", [(4096, 0.5), (1 << 20, 1e6), (4319216, 0.5)])
def test_adam_matches_torch(n, max_norm, cuda):
    p, g = _adam_case(n, n)
    tp = torch.nn.Parameter(torch.from_numpy(p.copy()))
    opt = oadam.OracleAdam([tp], lr=3e-4)
    L = native.lib()
    dp, dm_, dv = dev(p), empty(n), empty(n)
    step = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = empty(native.lib().ptcg_adam_workspace_floats())
    norm = empty(1)
    lr = lr_dev(3e-4)
    for it in range(3):
        gi = g * (1 + it)
        tp.grad = torch.from_numpy(gi.copy())
        tnorm = opt.step(max_norm)
        dg = dev(gi)
        native.check(L.ptcg_adam_step(P(dp), P(dg), P(dm_), P(dv), n, P(lr), 0.9, 0.999, 1e-8,
                                      max_norm, None, P(step), P(norm), P(ws), None))
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    assert step.item() == 3
    assert abs(norm.item() - float(tnorm)) <= 1e-6 * float(tnorm)
    m_ref, v_ref = opt.moments()
    assert rel_l2(dm_.cpu(), m_ref) < 1e-5
    assert rel_l2(dv.cpu(), v_ref) < 1e-5
    upd_gpu = dp.cpu().numpy() - p
    upd_ref = tp.detach().numpy() - p
    assert rel_l2(upd_gpu, upd_ref) < 1e-4


def test_adam_float_lr_entry_matches_double(cuda):
    """ptcg_adam_step_lrf reads the learning rate from a device float (the
    reference's lr_ptr); with an lr exact in both types the two entry points
    give the same bits."""
    n = 300000
    p, g = _adam_case(n, 17)
    L = native.lib()
    out = []
    for fn, lr in ((L.ptcg_adam_step, lr_dev(2.0 ** -12)),
                   (L.ptcg_adam_step_lrf, torch.tensor([2.0 ** -12], dtype=torch.float32, device="cuda"))):
        dp, dm_, dv, dg = dev(p), empty(n), empty(n), dev(g)
        step = torch.zeros(1, dtype=torch.int32, device="cuda")
        ws = empty(L.ptcg_adam_workspace_floats())
        for _ in range(2):
            native.check(fn(P(dp), P(dg), P(dm_), P(dv), n, P(lr), 0.9, 0.999, 1e-8, 0.5, None, P(step), None,
                            P(ws), None))
        torch.cuda.synchronize()
        out.append((dp.cpu().numpy(), dm_.cpu().numpy(), dv.cpu().numpy(), step.item()))
    for a, b in zip(out[0][:3], out[1][:3]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert out[0][3] == out[1][3] == 2


def test_adam_gate_zero_is_bit_exact_noop(cuda):
    n = 8192
    p, g = _adam_case(n, 5)
    g[7] = np.nan
    L = native.lib()
    dp, dm_, dv = dev(p), dev(np.full(n, 0.25, np.float32)), dev(np.full(n, 0.5, np.float32))
    step = torch.full((1,), 4, dtype=torch.int32, device="cuda")
    ws = empty(L.ptcg_adam_workspace_floats())
    gate = dev(np.zeros(1, np.float32))
    dg = dev(g)
    lr = lr_dev(1e-3)
    native.check(L.ptcg_adam_step(P(dp), P(dg), P(dm_), P(dv), n, P(lr), 0.9, 0.999, 1e-8, 0.5,
                                  P(gate), P(step), None, P(ws), None))
    torch.cuda.synchronize()
    assert np.array_equal(dp.cpu().numpy().view(np.uint32), p.view(np.uint32))
    assert torch.all(dm_ == 0.25) and torch.all(dv == 0.5) and step.item() == 4
    assert np.array_equal(dg.cpu().numpy().view(np.uint32), g.view(np.uint32))


def test_adam_first_step_is_lr_sign(cuda):
    n = 4096
    p, g = _adam_case(n, 9)
    L = native.lib()
    dp = dev(p)
    step = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = empty(L.ptcg_adam_workspace_floats())
    dg, dm_, dv = dev(g), empty(n), empty(n)
    lr = lr_dev(1e-3)
    native.check(L.ptcg_adam_step(P(dp), P(dg), P(dm_), P(dv), n, P(lr), 0.9, 0.999, 1e-8,
                                  1e6, None, P(step), None, P(ws), None))
    torch.cuda.synchronize()
    d = dp.cpu().numpy().astype(np.float64) - p
    # first Adam step in closed form: m_hat = g, v_hat = g^2
    g64 = g.astype(np.float64)
    assert np.allclose(d, -1e-3 * g64 / (np.abs(g64) + 1e-8), rtol=1e-4, atol=2e-10)


def _bf16(t):
    return t.to(torch.bfloat16).to(torch.float64)


BF16_CASES = [(37, 52, 300, 0, 0, 1), (130, 68, 64, 0, 0, 2), (256, 256, 256, 0, 0, 3), (200, 96, 40, 0, 1, 4),
              (64, 300, 256, 0, 1, 0), (768, 256, 20000, 1, 1, 0), (96, 36, 12, 1, 0, 0), (129, 132, 132, 0, 1, 5),
              (4096, 1024, 256, 0, 0, 2), (4096, 256, 1024, 0, 1, 0), (34000, 256, 256, 0, 0, 2),
              (300, 200, 48, 0, 0, 1), (64, 128, 16, 0, 1, 0), (1000, 136, 80, 1, 0, 7)]


@pytest.mark.parametrize("case", BF16_CASES, ids=lambda c: "M%d_N%d_K%d_at%d_bt%d_e%d" % c)
def test_gemm_bf16_products(case, cuda):
    """bf16 operands (round to nearest even), fp32 accumulation: equals the
    fp64 product of the bf16-rounded operands to fp32-accumulation accuracy."""
    M, N, K, a_t, b_t, epi = case
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(K, M, generator=g) if a_t else torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g) if b_t else torch.randn(N, K, generator=g)
    bias = torch.randn(N, generator=g)
    R = torch.randn(M, N, generator=g)
    C0 = torch.randn(M, N, generator=g)
    Am = _bf16(A.T if a_t else A)
    Bm = _bf16(B if b_t else B.T)
    acc = Am @ Bm
    ref2 = None
    if epi == 0: ref = acc
    elif epi == 1: ref = acc + bias.double()
    elif epi == 2:
        ref = acc + bias.double()
        ref2 = gelu(ref)
    elif epi == 3: ref = acc + bias.double() + R.double()
    elif epi == 4: ref = acc * gelu_grad(R.double())
    elif epi == 6:
        z = acc + bias.double()
        ref, ref2 = gelu_grad(z), gelu(z)
    elif epi == 7: ref = acc * R.double()
    else: ref = C0.double() + acc
    dA, dB, dbias, dR = dev(A), dev(B), dev(bias), dev(R)
    dC = dev(C0) if epi == 5 else empty(M, N)
    dC2 = empty(M, N)
    ws = empty(32 << 20)
    native.check(native.lib().ptcg_kernel_gemm_bf16(M, N, K, P(dA), M if a_t else K, a_t, P(dB), N if b_t else K, b_t,
                                                    P(dC), N, epi, P(dbias), P(dR), N, P(dC2), N, P(ws), ws.numel(),
                                                    None))
    torch.cuda.synchronize()
    got = dC.cpu().double()
    assert rel_l2(got, ref) < 1e-5, rel_l2(got, ref)
    if ref2 is not None:
        assert rel_l2(dC2.cpu().double(), ref2) < 1e-5
    # and it is a bf16 product, not the fp32 one
    exact = (A.T if a_t else A).double() @ (B if b_t else B.T).double()
    if epi == 0:
        assert rel_l2(got, exact) > 1e-4


@pytest.mark.parametrize("rows,inp,out", [(6000, 256, 768), (1573, 128, 64), (100, 64, 36), (40000, 1024, 256),
                                          (37, 256, 256)])
def test_gemm_weight_grad_bf16_with_bias_sums(rows, inp, out, cuda):
    """bf16 weight gradient: dW equals the fp64 product of the bf16-rounded
    dY and X; the fused bias sums add the unrounded fp32 dY."""
    g = torch.Generator().manual_seed(rows + 3 * inp)
    dY = torch.randn(rows, out, generator=g)
    X = torch.randn(rows, inp, generator=g)
    d_dY, d_X, dW, db = dev(dY), dev(X), empty(out, inp), empty(out)
    ws = empty(32 << 20)
    native.check(native.lib().ptcg_kernel_gemm_dw_bf16(rows, inp, out, P(d_dY), out, P(d_X), inp, P(dW), P(db),
                                                       P(ws), ws.numel(), None))
    torch.cuda.synchronize()
    refW = _bf16(dY).T @ _bf16(X)
    refb = dY.double().sum(0)
    assert rel_l2(dW.cpu().double(), refW) < 1e-5
    assert rel_l2(db.cpu().double(), refb) < 1e-5
    assert rel_l2(dW.cpu().double(), dY.double().T @ X.double()) > 1e-4


# ---- products on bf16-stored operands (the mixed-precision variant's activations)
BS_CASES = [
    # M, N, K, epi, out_bf16
    (37, 52, 256, 0, 0), (300, 200, 64, 1, 1), (256, 256, 256, 3, 0), (130, 1024, 256, 6, 1),
    (4096, 256, 1024, 7, 1), (1000, 768, 256, 1, 1), (33000, 256, 256, 3, 0), (512, 256, 768, 0, 1),
    (129, 136, 40, 0, 0), (200, 96, 1032, 7, 1),
]


def _bf16_bits(t):
    """torch tensor -> (device bf16 tensor, its float64 value)."""
    b = t.to(torch.bfloat16)
    return b.to("cuda"), b.to(torch.float64)


@pytest.mark.parametrize("case", BS_CASES, ids=lambda c: "M%d_N%d_K%d_e%d_ob%d" % c)
def test_gemm_bf16_operands(case, cuda):
    """C = epi(A B^T) with A, B stored in bf16: fp32 outputs within relative L2
    1e-5 of the fp64 product of the same bf16 values; bf16 outputs within one
    bf16 rounding (2^-8 relative) of the fp64 result elementwise, plus 2^-20 of
    the output's largest magnitude (the fp32 accumulation error, which decides
    the rounding where acc + bias cancels to near zero)."""
    M, N, K, epi, ob = case
    g = torch.Generator().manual_seed(7 * M + N + K)
    dA, A = _bf16_bits(torch.randn(M, K, generator=g))
    dB, B = _bf16_bits(torch.randn(N, K, generator=g))
    bias = torch.randn(N, generator=g)
    Rf = torch.randn(M, N, generator=g)
    acc = A @ B.T
    ref2 = None
    dR = None
    if epi == 0: ref = acc
    elif epi == 1: ref = acc + bias.double()
    elif epi == 3:
        ref = acc + bias.double() + Rf.double()
        dR = dev(Rf)
    elif epi == 6:
        z = acc + bias.double()
        ref, ref2 = gelu_grad(z), gelu(z)
    elif epi == 7:
        dR, Rb = _bf16_bits(Rf)
        ref = acc * Rb
    odt = torch.bfloat16 if ob else torch.float32
    dC = torch.zeros(M, N, dtype=odt, device="cuda")
    dC2 = torch.zeros(M, N, dtype=odt, device="cuda")
    native.check(native.lib().ptcg_kernel_gemm_bs(M, N, K, P(dA), K, P(dB), K, P(dC), N, epi, ob, P(dev(bias)),
                                                  P(dR), N, P(dC2), N, None))
    torch.cuda.synchronize()
    outs = [(dC, ref)] + ([(dC2, ref2)] if ref2 is not None else [])
    for d, r in outs:
        got = d.cpu().double()
        if ob:
            # one bf16 rounding of the fp32 result; fp32 accumulation error is far smaller
            tol = 2.0 ** -8 * r.abs() + 2.0 ** -20 * float(r.abs().max())
            assert torch.all((got - r).abs() <= tol), ((got - r).abs() - tol).max()
            assert rel_l2(got, r) < 4e-3
        else:
            assert rel_l2(got, r) < 1e-5, rel_l2(got, r)


def test_gemm_bf16_operands_rejects_bad_shapes(cuda):
    a = torch.zeros(64, 36, dtype=torch.bfloat16, device="cuda")
    c = torch.zeros(64, 64, device="cuda")
    with pytest.raises(RuntimeError, match="multiples of 8"):
        native.check(native.lib().ptcg_kernel_gemm_bs(64, 64, 36, P(a), 36, P(a), 36, P(c), 64, 0, 0, None, None,
                                                      0, None, 0, None))
    with pytest.raises(RuntimeError, match="not built"):
        b = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda")
        native.check(native.lib().ptcg_kernel_gemm_bs(64, 64, 64, P(b), 64, P(b), 64, P(c), 64, 1, 0, P(c), None,
                                                      0, None, 0, None))


@pytest.mark.parametrize("rows,inp,out", [(6000, 256, 768), (1576, 128, 64), (104, 64, 40), (150000, 256, 1024),
                                          (37, 256, 256), (40000, 1024, 256), (1, 8, 8)])
def test_gemm_weight_grad_bf16_operands(rows, inp, out, cuda):
    """dW = dY^T X and db = column sums of dY with dY, X stored in bf16: both
    within relative L2 1e-5 of the fp64 values of the same bf16 inputs, and
    bit-identical on a second call (fixed-order split sums)."""
    g = torch.Generator().manual_seed(rows + 5 * inp + out)
    d_dY, dY = _bf16_bits(torch.randn(rows, out, generator=g))
    d_X, X = _bf16_bits(torch.randn(rows, inp, generator=g))
    ws = empty(32 << 20)
    res = []
    for _ in range(2):
        dW, db = empty(out, inp), empty(out)
        native.check(native.lib().ptcg_kernel_gemm_dw_bs(rows, inp, out, P(d_dY), out, P(d_X), inp, P(dW), P(db),
                                                         P(ws), ws.numel(), None))
        torch.cuda.synchronize()
        res.append((dW.cpu(), db.cpu()))
    assert rel_l2(res[0][0].double(), dY.T @ X) < 1e-5
    assert rel_l2(res[0][1].double(), dY.sum(0)) < 1e-5
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
