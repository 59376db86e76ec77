// Model driver: weight binding, activation arena, forward and backward.
//
// Mirrors the reference's PTCG Encoder plugin (native/model/ptcg_model3.cu
// ptcg_forward_core :246-369, blk_fwd :12-40, blk_bwd :44-95;
// ptcg_model4.cu ptcg_backward_core :10-190; ptcg_model2.cu tables_fwd /
// tables_bwd :422-485) with a different kernel plan:
//   * GEMM epilogues carry bias, GELU, residual add and the GELU backward,
//     so there are no separate bias / gelu / add kernels; a GELU layer's
//     forward keeps gelu'(z) in place of the pre-activation z (the only
//     thing the backward needs of z), so its backward is one multiply in
//     the epilogue of the next layer's dX product;
//   * attention is one fused kernel per direction (no (N,H,L,L) tensor);
//   * concat inputs are written in place by the producing GEMMs (leading
//     dimension = concat width) — g/dvec into the bcast input, opt_card /
//     opt_attack into q_in, q into the score input; the static / text
//     columns of the table-chain inputs are written once at upload;
//   * every activation the backward needs is kept (LayerNorm outputs, qkv,
//     attention context, GELU derivatives and outputs), so the backward
//     recomputes nothing but the attention probabilities.
// Two switches select the model variant: tables (learned card / attack
// tables, or the static-table chain rebuilt every forward) and critic (blind
// value head, or the oracle critic block with the blind value and belief aux
// heads trained by losses injected in the backward).
// Grads are overwritten on every backward (ptcg_model4.cu:15-21).
#include "model.h"

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

struct BlockP {
    float *ln1w, *ln1b, *qkvw, *qkvb, *projw, *projb, *ln2w, *ln2b, *f1w, *f1b, *f2w, *f2b;
};
// per-layer activations; ffp = gelu'(z) and ffa = gelu(z) of the FFN's
// first product z (every GELU layer keeps its derivative, not z)
struct BlockA {
    float *ln1, *mu1, *rs1, *qkv, *ctx, *lse, *xmid, *ln2, *mu2, *rs2, *ffp, *ffa;
};
// bf16 variant: bf16 copies of a block's weight matrices, W (out, in) for the
// forward products and W^T (in, out) for the backward's dX
struct BlockW {
    __bf16 *qkv, *qkvT, *proj, *projT, *f1, *f1T, *f2, *f2T;
};

struct PtcgModel {
    PtcgDims dm;
    DimsX dx;
    ObsOff off;
    std::vector<ParamDef> defs;
    std::vector<long> offs;
    long arena = 0;
    float* P = nullptr;
    float* Gr = nullptr;
    // card / attack vectors the gathers read, and where their gradients go:
    // the learned tables and their grads, or the table chain's outputs and
    // scratch gradients that the chain's backward consumes
    float *card = nullptr, *att = nullptr, *dcard = nullptr, *datt = nullptr;
    float *zemb, *oemb, *tp_w, *tp_b, *readout, *g1_w, *g1_b, *g2_w, *g2_b, *semb, *cemb, *d1_w, *d1_b,
        *d2_w, *d2_b, *bc_w, *bc_b;
    std::vector<BlockP> blk;
    float *lnf_w, *lnf_b, *temb, *oc_w, *oc_b, *oa_w, *oa_b, *q1_w, *q1_b, *q2_w, *q2_b, *s1_w,
        *s1_b, *s2_w, *s2_b, *v1_w, *v1_b, *v2_w, *v2_b;
    // static-table chain weights (tables == 1)
    float *cid_emb = nullptr, *aid_emb, *sid_emb, *am_w, *am_b, *sm_w, *sm_b, *cln_w, *cln_b, *c1_w, *c1_b,
        *c3_w, *c3_b;
    // oracle critic + aux heads (critic == 1)
    float *op_w = nullptr, *op_b, *cread, *ov1_w, *ov1_b, *ov2_w, *ov2_b, *ah_w, *ah_b, *ap_w, *ap_b;
    BlockP cblk;
    // static tables and the chain's batch-independent buffers (own allocation)
    char* tmem = nullptr;
    int *card_attacks, *card_skills, *a_amax, *s_amax;
    float *att_in, *att_lin, *att_tab, *sk_in, *sk_lin, *sk_tab, *card_in, *c_mu, *c_rs, *card_ln, *card_h1,
        *card_g1, *card_vec;
    float *d_card_vec, *d_att_tab, *d_sk_tab, *d_card_h, *d_card_ln, *d_card_in, *d_att_lin, *d_sk_lin;
    // activations (train: every layer's kept for the backward; rollout:
    // one block's worth reused by every layer, no backward buffers)
    int N = 0;
    bool train = true;
    int prec = 0;   // GEMM products: 0 fp32, 1 bf16 operands with fp32 accumulation
    // compact trunk layout (blind-critic models): only READOUT, valid tokens
    // and pointer targets are trunk rows; *Tr = their count (device).
    // Default: the count is read back once per forward (pinned rows_h) and
    // every trunk launch is sized for exactly those rows (rows, Tdev null).
    // sync_free: no host read-back, so the step stays stream-ordered and can
    // be captured in a HIP graph; launches are sized for N * l_seq rows and
    // stop at the device count (rows = N * l_seq, Tdev = Tr).
    bool compact = false;
    bool sync_free = false;
    int *c_act = nullptr, *c_cnt, *c_off, *c_map, *c_rsam, *c_rpos;
    const int* Tr = nullptr;
    int* rows_h = nullptr;   // pinned: [trunk rows, option rows]
    int rows = 0;
    const int* Tdev = nullptr;
    // masked-option skipping (a loss that masks them, as the PPO loss does):
    // the option scorer runs only each sample's legal options (all of them
    // when none is legal), stored contiguously per sample (o_off, o_row);
    // masked slots of the output read 0.  orows / Odev: host / device count,
    // as rows / Tdev above.  skip_fwd: the mode the last forward ran in.
    bool skip_masked = false, skip_fwd = false;
    int *o_cnt = nullptr, *o_off = nullptr, *o_row = nullptr;
    int orows = 0;
    const int* Odev = nullptr;
    float* rd_buf = nullptr;
    char* mem = nullptr;
    size_t mem_bytes = 0;
    float *tok_cat, *tokp, *glob_in, *g1, *g1a, *dec_in, *d1, *d1a, *gd, *bc, *keep;
    std::vector<float*> x;
    std::vector<BlockA> ba;
    float *h, *lnf_mu, *lnf_rs;
    float *ocard, *oatt, *q_in, *q1, *q1a, *sc_in, *s1, *s1a, *val_in, *v1, *v1a, *out;
    float *dxa, *dxb, *dffn, *dln, *dqkv, *dctx, *dsc, *ds1, *dq, *dq1, *dqin, *docard, *doatt,
        *dvin, *dv1, *dgd, *dd1, *dg1, *ddec, *dtokp, *dtokcat, *dbc;
    // oracle critic / aux activations and scratch
    float *otok_in, *otok, *ckeep, *xc, *xco, *ov_in, *ov1, *ov1a, *bv, *hand_lin, *prize_all;
    BlockA cba;
    // bf16 variant (prec 1): the blocks keep ln1 / qkv / ctx / ln2 / ffp / ffa
    // and the backward's dffn / dctx / dqkv in bf16 (the residual stream, the
    // LayerNorm statistics and the parameter gradients stay fp32); weight
    // copies refreshed every forward; dAh / dCh: bf16 copies of the residual
    // gradients dA / dC (written by the LayerNorm backward that produces them)
    std::vector<BlockW> bw;
    BlockW cbw{};
    float *dAh = nullptr, *dCh = nullptr;
    // the blocks' weight gradients run on a side stream (wg_s) concurrently
    // with the backward's critical path (dX, LayerNorm, attention); wg_ev[0]
    // forks the side stream off the main one, wg_ev[1..4] mark the side
    // stream's FFN2 / FFN1 / out-projection / QKV weight gradient of the
    // latest block done (wg_rec: recorded in this backward); ws2 is the side
    // stream's split-K workspace; wg_serial (set per backward while a launch
    // profile is open) keeps them on the main stream, so that every timed
    // launch runs alone.  The heads' and trunk input's weight gradients go to
    // the side stream too (ldw_side), wg_ev[5] marking the latest of them.
    // In a training forward wg_ev[6] / wg_ev[7] mark the side stream's
    // per-sample MLPs and option-row projections, wg_ev[8] the main stream's
    // row compaction (model_forward).
    hipStream_t wg_s = nullptr;
    bool wg_serial = false;
    hipEvent_t wg_ev[9] = {};
    bool wg_rec[9] = {};
    float* ws2 = nullptr;
    long ws2_floats = 0;
    // the trunk attention backward's dS scratch (training only)
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    float *d_hand, *d_prize, *d_blind, *dxc, *dxc2, *dotok, *dotok_in, *dov1, *dovin;
    int* aux_cnt;
    // order-independent table scatters: fixed-point accumulators (zero
    // between sites), per-block maxima, per-table scales
    DetCtx det{};
    const float* ret = nullptr;
    float* ws = nullptr;
    long ws_floats = 0;
    const float* obs = nullptr;
    const int32_t* idx = nullptr;

    float* G(const float* p) const { return Gr + (p - P); }
};

// ------------------------------------------------------------ helpers
// Y = epi(X W^T + b) with workspace ws for split-K / tail partials
static int lin_ws(const PtcgModel* m, float* ws, long ws_floats, const float* X, long ldx, const float* W,
                  const float* b, float* Y, long ldy, int rows, int in, int out, int epi, const float* R, long ldr,
                  float* Y2, long ldy2, hipStream_t s, const int* Mdev = nullptr) {
    GemmArgs g{};
    g.prec = m->prec;
    g.Mdev = Mdev;
    g.M = rows; g.N = out; g.K = in;
    g.A = X; g.lda = ldx; g.a_t = 0;
    g.B = W; g.ldb = in; g.b_t = 0;
    g.C = Y; g.ldc = ldy;
    g.bias = b; g.R = R; g.ldr = ldr; g.C2 = Y2; g.ldc2 = ldy2;
    g.epi = epi;
    return pt_gemm(g, ws, ws_floats, s);
}
static int lin(const PtcgModel* m, const float* X, long ldx, const float* W, const float* b, float* Y, long ldy,
               int rows, int in, int out, int epi, const float* R, long ldr, float* Y2, long ldy2,
               hipStream_t s, const int* Mdev = nullptr) {
    return lin_ws(m, m->ws, m->ws_floats, X, ldx, W, b, Y, ldy, rows, in, out, epi, R, ldr, Y2, ldy2, s, Mdev);
}
static int linf(const PtcgModel* m, const float* X, const float* W, const float* b, float* Y, int rows, int in,
                int out, int epi, const float* R, float* Y2, hipStream_t s, const int* Mdev = nullptr) {
    return lin(m, X, in, W, b, Y, out, rows, in, out, epi, R, out, Y2, out, s, Mdev);
}
// A LayerNorm that reads a residual product's output: weights, output and
// statistics (eps 1e-5, rows of d)
struct LnOut {
    const float* w; const float* b; float* y; float* mu; float* rs;
    int ybf = 0;   // y stored in bf16 (the mixed-precision blocks' LayerNorm outputs)
};
// Y = X W^T + b + R (rows x out, out = d), then ln(Y): one fused launch when
// the shape fits it (fp32, d = 256) and K < 1024, else the product and
// pt_ln_fwd.  The fused kernel's 32-row tiles each re-read all of W, so its
// cost grows with K faster than the 128 x 128-tile product's: measured alone
// (fused vs product + LayerNorm), 37.4k rows x K 256: 67 vs ~89 us, K 512:
// 119 vs ~133, K 1024: 231 vs ~213.  In the CORE step (FFN2 at K 1024
// unfused) +0.4% replayed, +0.8% stream-launched; the reference variant's
// FFN2 at K 512 x 82.4k rows (280 vs ~258 alone) ran 0.3% slower unfused in
// its step, so it stays fused.  Both give the same bits.
static int lin_resid_ln(const PtcgModel* m, const float* X, const float* W, const float* b, float* Y, int rows,
                        int in, int out, const float* R, const LnOut& ln, hipStream_t s, const int* Mdev) {
    GemmArgs g{};
    g.prec = m->prec;
    g.Mdev = Mdev;
    g.M = rows; g.N = out; g.K = in;
    g.A = X; g.lda = in;
    g.B = W; g.ldb = in;
    g.C = Y; g.ldc = out;
    g.bias = b; g.R = R; g.ldr = out;
    g.epi = EPI_BIAS_RESID;
    if (pt_gemm_resid_ln_fits(g) && in < 1024)
        return pt_gemm_resid_ln(g, ln.w, ln.b, ln.y, out, ln.mu, ln.rs, s, ln.ybf);
    PT_TRY(pt_gemm(g, m->ws, m->ws_floats, s));
    return pt_ln_fwd(Y, out, ln.w, ln.b, ln.y, out, ln.mu, ln.rs, rows, out, s, Mdev, ln.ybf);
}
// dX = dY W[:, :in] : dY (rows, out) ld lddy ; W (out, ldw) ; dX (rows, in) ld lddx
static int ldxw_(const PtcgModel* m, const float* dY, long lddy, const float* W, long ldw, float* dX, long lddx,
                 int rows, int in, int out, int epi, const float* R, long ldr, hipStream_t s,
                 const int* Mdev = nullptr) {
    GemmArgs g{};
    g.prec = m->prec;
    g.Mdev = Mdev;
    g.M = rows; g.N = in; g.K = out;
    g.A = dY; g.lda = lddy; g.a_t = 0;
    g.B = W; g.ldb = ldw; g.b_t = 1;
    g.C = dX; g.ldc = lddx;
    g.R = R; g.ldr = ldr;
    g.epi = epi;
    return pt_gemm(g, m->ws, m->ws_floats, s);
}
// dX = dY W : dY (rows, out) ld lddy ; W (out, in) ; dX (rows, in) ld lddx
static int ldx_(const PtcgModel* m, const float* dY, long lddy, const float* W, float* dX, long lddx, int rows,
                int in, int out, int epi, const float* R, long ldr, hipStream_t s, const int* Mdev = nullptr) {
    return ldxw_(m, dY, lddy, W, in, dX, lddx, rows, in, out, epi, R, ldr, s, Mdev);
}
// dW = dY^T X (overwrite), db = colsum dY (fused into the product)
// (side = true: on the side stream's workspace)
static int ldw_(PtcgModel* m, const float* dY, long lddy, const float* X, long ldxx, float* dW,
                float* db, int rows, int in, int out, hipStream_t s, const int* Kdev = nullptr, bool side = false) {
    GemmArgs g{};
    g.Kdev = Kdev;
    g.M = out; g.N = in; g.K = rows;
    g.A = dY; g.lda = lddy; g.a_t = 1;
    g.B = X; g.ldb = ldxx; g.b_t = 1;
    g.C = dW; g.ldc = in;
    g.epi = EPI_STORE;
    g.dbias = db;
    g.prec = m->prec;
    return pt_gemm(g, side ? m->ws2 : m->ws, side ? m->ws2_floats : m->ws_floats, s);
}

// bf16-operand products (GemmArgs::bs) of the bf16 variant's blocks:
// Y = epi(X Wb^T), X (rows, in) and Wb (out, in) bf16; obf: Y (and Y2) bf16;
// R at leading dimension out (bf16 for EPI_MUL, fp32 for EPI_BIAS_RESID).
// The backward's dX = dY W is the same product with Wb = W^T (in, out).
static int blin(const PtcgModel* m, const float* X, int in, const __bf16* Wb, const float* b, float* Y, int out,
                int rows, int epi, bool obf, const float* R, float* Y2, hipStream_t s, const int* Mdev) {
    GemmArgs g{};
    g.prec = 1; g.bs = 1; g.obf = obf ? 1 : 0;
    g.Mdev = Mdev;
    g.M = rows; g.N = out; g.K = in;
    g.A = X; g.lda = in;
    g.B = reinterpret_cast<const float*>(Wb); g.ldb = in;
    g.C = Y; g.ldc = out;
    g.bias = b; g.R = R; g.ldr = out; g.C2 = Y2; g.ldc2 = out;
    g.epi = epi;
    return pt_gemm(g, m->ws, m->ws_floats, s);
}
// dW (out, in) = dY^T X, db = column sums of dY, with dY (rows, out) and X (rows, in) bf16
// (on the side stream's workspace)
// blin's residual product (bf16 X and weight copy, fp32 Y and R) followed by
// ln(Y): one fused launch when the shape fits it, else the product and the
// LayerNorm
static int blin_resid_ln(const PtcgModel* m, const float* X, int in, const __bf16* Wb, const float* b, float* Y,
                         int out, int rows, const float* R, const LnOut& ln, hipStream_t s, const int* Mdev) {
    GemmArgs g{};
    g.prec = 1; g.bs = 1;
    g.Mdev = Mdev;
    g.M = rows; g.N = out; g.K = in;
    g.A = X; g.lda = in;
    g.B = reinterpret_cast<const float*>(Wb); g.ldb = in;
    g.C = Y; g.ldc = out;
    g.bias = b; g.R = R; g.ldr = out;
    g.epi = EPI_BIAS_RESID;
    if (pt_gemm_resid_ln_fits(g)) return pt_gemm_resid_ln(g, ln.w, ln.b, ln.y, out, ln.mu, ln.rs, s, ln.ybf);
    PT_TRY(pt_gemm(g, m->ws, m->ws_floats, s));
    return pt_ln_fwd(Y, out, ln.w, ln.b, ln.y, out, ln.mu, ln.rs, rows, out, s, Mdev, ln.ybf);
}
// blin's dX product dln = dY W (dY bf16 (rows, in), weight copy W^T (D, in))
// followed by the LayerNorm backward of dln: one fused launch when the shape
// fits it, else the product and pt_ln_bwd
static int blin_dx_lnbwd(PtcgModel* m, const float* dY, int in, const __bf16* WT, int rows, const float* x,
                         const float* lnw, const float* mu, const float* rs, const float* dres, float* dx,
                         float* dw, float* db, float* dxh, hipStream_t s, const int* Mdev) {
    const int D = m->dm.d;
    GemmArgs g{};
    g.prec = 1; g.bs = 1;
    g.Mdev = Mdev;
    g.M = rows; g.N = D; g.K = in;
    g.A = dY; g.lda = in;
    g.B = reinterpret_cast<const float*>(WT); g.ldb = in;
    g.epi = EPI_STORE;
    if (pt_dx_lnbwd_fits(g)) return pt_dx_lnbwd(g, x, lnw, mu, rs, dres, dx, dxh, dw, db, m->ws, m->ws_floats, s);
    PT_TRY(blin(m, dY, in, WT, nullptr, m->dln, D, rows, EPI_STORE, false, nullptr, nullptr, s, Mdev));
    return pt_ln_bwd(m->dln, D, x, D, lnw, mu, rs, dres, D, dx, D, dw, db, rows, D, m->ws, m->ws_floats, s, Mdev,
                     dxh);
}
static int bldw(PtcgModel* m, const float* dY, int out, const float* X, int in, float* dW, float* db, int rows,
                hipStream_t s, const int* Kdev) {
    GemmArgs g{};
    g.prec = 1; g.bs = 1;
    g.Kdev = Kdev;
    g.M = out; g.N = in; g.K = rows;
    g.A = dY; g.lda = out; g.a_t = 1;
    g.B = X; g.ldb = in; g.b_t = 1;
    g.C = dW; g.ldc = in; g.epi = EPI_STORE;
    g.dbias = db;
    return pt_gemm(g, m->ws2, m->ws2_floats, s);
}

// side-stream ordering: mark = record the main stream's work so far;
// take = the side stream waits for the last mark; done(e) = mark the side
// stream's work so far as event e; after(e) = the main stream waits for
// event e (if this backward recorded it).  A weight gradient is marked once
// its dY exists, and taken after the main stream's next product is enqueued:
// the same dependencies, but in a captured step the dX product is the first
// child of the node before it, which is the one graph replay keeps on that
// node's queue (captured the other way round, the replays ran the dX product
// after the weight gradient on one queue)
static int wg_mark(PtcgModel* m, hipStream_t s) {
    if (m->wg_serial) return PTCG_OK;
    PT_HIP(hipEventRecord(m->wg_ev[0], s));
    return PTCG_OK;
}
static int wg_take(PtcgModel* m) {
    if (m->wg_serial) return PTCG_OK;
    PT_HIP(hipStreamWaitEvent(m->wg_s, m->wg_ev[0], 0));
    return PTCG_OK;
}
static int wg_done(PtcgModel* m, int e) {
    if (m->wg_serial) return PTCG_OK;
    PT_HIP(hipEventRecord(m->wg_ev[e], m->wg_s));
    m->wg_rec[e] = true;
    return PTCG_OK;
}
static int wg_after(PtcgModel* m, int e, hipStream_t s) {
    if (m->wg_rec[e]) PT_HIP(hipStreamWaitEvent(s, m->wg_ev[e], 0));
    return PTCG_OK;
}

// A weight gradient of the heads or the trunk input on the side stream,
// after the last wg_mark (placed once its dY is written; the main stream's
// dX product is enqueued between the two); its dY and X are not rewritten
// later in the backward, and the backward joins wg_ev[5] before it returns
static int ldw_side(PtcgModel* m, const float* dY, long lddy, const float* X, long ldxx, float* dW, float* db,
                    int rows, int in, int out, hipStream_t s, const int* Kdev = nullptr) {
    if (m->wg_serial) return ldw_(m, dY, lddy, X, ldxx, dW, db, rows, in, out, s, Kdev);
    PT_TRY(wg_take(m));
    PT_TRY(ldw_(m, dY, lddy, X, ldxx, dW, db, rows, in, out, m->wg_s, Kdev, true));
    return wg_done(m, 5);
}

// a dot head's weight gradient (pt_head_dot_dw) on the side stream, after the
// last wg_mark, like ldw_side: grad and X are not rewritten later in the
// backward
static int head_dw_side(PtcgModel* m, const float* grad, int per, long ldg, int col0, const float* X, int rows,
                        int K, float* dw, float* db, hipStream_t s, const int* rmap = nullptr,
                        const int* rows_dev = nullptr) {
    if (m->wg_serial)
        return pt_head_dot_dw(grad, per, ldg, col0, X, rows, K, dw, db, m->ws, m->ws_floats, s, rmap, rows_dev);
    PT_TRY(wg_take(m));
    PT_TRY(pt_head_dot_dw(grad, per, ldg, col0, X, rows, K, dw, db, m->ws2, m->ws2_floats, m->wg_s, rmap, rows_dev));
    return wg_done(m, 5);
}

// refresh the blocks' bf16 weight copies from the fp32 masters
static int bf16_refresh(PtcgModel* m, hipStream_t s) {
    BfWeightSet ws;
    const int D = m->dm.d, F = m->dm.ffn, nl = (int)m->blk.size();
    const int nb = nl + (m->dm.critic == 1 ? 1 : 0);
    for (int i = 0; i < nb; ++i) {
        const BlockP& p = i < nl ? m->blk[i] : m->cblk;
        const BlockW& w = i < nl ? m->bw[i] : m->cbw;
        const BfWeight mats[4] = {{p.qkvw, w.qkv, w.qkvT, 3 * D, D, 0}, {p.projw, w.proj, w.projT, D, D, 0},
                                  {p.f1w, w.f1, w.f1T, F, D, 0}, {p.f2w, w.f2, w.f2T, D, F, 0}};
        for (const BfWeight& bwm : mats) {
            if (ws.n == BF_MAX_W) {
                PT_TRY(pt_bf16_weights(ws, s));
                ws.n = 0;
            }
            ws.m[ws.n++] = bwm;
        }
    }
    if (ws.n) PT_TRY(pt_bf16_weights(ws, s));
    return PTCG_OK;
}

struct Carver {
    char* base; size_t off = 0;
    float* take(size_t floats) {
        off = (off + 255) & ~(size_t)255;
        float* p = base ? reinterpret_cast<float*>(base + off) : nullptr;
        off += floats * sizeof(float);
        return p;
    }
    __bf16* take_bf(size_t n) { return reinterpret_cast<__bf16*>(take((n + 1) / 2)); }
};

// ------------------------------------------------------------ lifecycle
extern "C" int ptcg_model_create(const PtcgDims* dims, PtcgModel** out) {
    PT_REQUIRE(dims && out, "model_create: null argument");
    PtcgDims d = *dims;
    PT_REQUIRE(d.tables == 0 || d.tables == 1, "model_create: unknown tables mode %d", d.tables);
    PT_REQUIRE(d.critic == 0 || d.critic == 1, "model_create: unknown critic mode %d", d.critic);
    PT_REQUIRE(d.d % d.heads == 0, "model_create: d=%d not divisible by heads=%d", d.d, d.heads);
    PT_REQUIRE(d.n_opt <= 64, "model_create: n_opt=%d > 64 unsupported", d.n_opt);
    PT_REQUIRE(d.d % 4 == 0 && d.d_c % 4 == 0 && d.d_a % 4 == 0 && d.g % 4 == 0 && d.ffn % 4 == 0 &&
               d.tok_f % 4 == 0 && d.opt_f % 4 == 0 && d.global_f % 4 == 0,
               "model_create: widths must be multiples of 4");
    PT_REQUIRE(pt_attn_supported(d.l_tok + 1, d.d / d.heads),
               "model_create: attention shape L=%d Dh=%d unsupported", d.l_tok + 1, d.d / d.heads);
    if (d.critic == 1) {
        PT_REQUIRE(d.oracle_f == 2 * PT_N_HAND + 3 * PT_N_SPLIT + 2 * PT_N_PRIZE,
                   "model_create: the oracle critic needs a %d-float oracle block, got %d",
                   2 * PT_N_HAND + 3 * PT_N_SPLIT + 2 * PT_N_PRIZE, d.oracle_f);
        const int lc = d.l_tok + 2 + PT_N_HAND + PT_N_SPLIT + PT_N_PRIZE;
        PT_REQUIRE(pt_attn_supported(lc, d.d / d.heads),
                   "model_create: critic attention shape L=%d Dh=%d unsupported", lc, d.d / d.heads);
        PT_REQUIRE(d.n_cards <= 8192, "model_create: n_cards=%d too large for the aux targets", d.n_cards);
    }
    PtcgModel* m = new PtcgModel();
    m->dm = d;
    m->dx = pt_dims_x(d);
    m->off = pt_obs_offsets(d);
    ParamDef tmp[256];
    int np = pt_param_table(d, tmp, 256);
    if (np < 0) { delete m; return PTCG_ERR_ARG; }
    m->defs.assign(tmp, tmp + np);
    long off = 0;
    for (auto& p : m->defs) {
        off = (off + 3) & ~3L;
        m->offs.push_back(off);
        off += p.rows * (p.cols > 0 ? p.cols : 1);
    }
    m->arena = (off + 3) & ~3L;
    *out = m;
    return PTCG_OK;
}

long pt_model_arena(const PtcgModel* m) { return m->arena; }

static void bind_block(const std::map<std::string, float*>& byname, const std::string& p, BlockP& b) {
    auto get = [&](const std::string& n) -> float* {
        auto it = byname.find(n);
        return it == byname.end() ? nullptr : it->second;
    };
    b.ln1w = get(p + "ln1.weight"); b.ln1b = get(p + "ln1.bias");
    b.qkvw = get(p + "qkv.weight"); b.qkvb = get(p + "qkv.bias");
    b.projw = get(p + "proj.weight"); b.projb = get(p + "proj.bias");
    b.ln2w = get(p + "ln2.weight"); b.ln2b = get(p + "ln2.bias");
    b.f1w = get(p + "ffn.0.weight"); b.f1b = get(p + "ffn.0.bias");
    b.f2w = get(p + "ffn.2.weight"); b.f2b = get(p + "ffn.2.bias");
}

extern "C" int ptcg_model_bind(PtcgModel* m, float* params, float* grads) {
    PT_REQUIRE(m && params && grads, "model_bind: null argument");
    PT_REQUIRE(((uintptr_t)params & 15) == 0 && ((uintptr_t)grads & 15) == 0,
               "model_bind: arenas must be 16 B aligned");
    m->P = params;
    m->Gr = grads;
    std::map<std::string, float*> byname;
    for (size_t i = 0; i < m->defs.size(); ++i) byname[m->defs[i].name] = params + m->offs[i];
    auto get = [&](const std::string& n) -> float* {
        auto it = byname.find(n);
        return it == byname.end() ? nullptr : it->second;
    };
    if (m->dm.tables == 0) {
        m->card = get("card_table"); m->att = get("attack_table");
        PT_REQUIRE(m->card && m->att, "model_bind: parameter table incomplete");
        m->dcard = m->G(m->card); m->datt = m->G(m->att);
    } else {
        m->cid_emb = get("card_id_emb.weight"); m->aid_emb = get("attack_id_emb.weight");
        m->sid_emb = get("skill_id_emb.weight");
        m->am_w = get("attack_mlp.0.weight"); m->am_b = get("attack_mlp.0.bias");
        m->sm_w = get("skill_mlp.0.weight"); m->sm_b = get("skill_mlp.0.bias");
        m->cln_w = get("card_mlp.0.weight"); m->cln_b = get("card_mlp.0.bias");
        m->c1_w = get("card_mlp.1.weight"); m->c1_b = get("card_mlp.1.bias");
        m->c3_w = get("card_mlp.3.weight"); m->c3_b = get("card_mlp.3.bias");
        PT_REQUIRE(m->cid_emb && m->c3_b, "model_bind: parameter table incomplete");
    }
    m->zemb = get("zone_emb.weight"); m->oemb = get("owner_emb.weight");
    m->tp_w = get("token_proj.weight"); m->tp_b = get("token_proj.bias");
    m->readout = get("readout");
    m->g1_w = get("global_mlp.0.weight"); m->g1_b = get("global_mlp.0.bias");
    m->g2_w = get("global_mlp.2.weight"); m->g2_b = get("global_mlp.2.bias");
    m->semb = get("sel_type_emb.weight"); m->cemb = get("ctx_emb.weight");
    m->d1_w = get("dec_mlp.0.weight"); m->d1_b = get("dec_mlp.0.bias");
    m->d2_w = get("dec_mlp.2.weight"); m->d2_b = get("dec_mlp.2.bias");
    m->bc_w = get("bcast.weight"); m->bc_b = get("bcast.bias");
    m->blk.resize(m->dm.layers);
    for (int i = 0; i < m->dm.layers; ++i) bind_block(byname, "blocks." + std::to_string(i) + ".", m->blk[i]);
    m->lnf_w = get("ln_f.weight"); m->lnf_b = get("ln_f.bias");
    m->temb = get("opt_type_emb.weight");
    m->oc_w = get("opt_card.weight"); m->oc_b = get("opt_card.bias");
    m->oa_w = get("opt_attack.weight"); m->oa_b = get("opt_attack.bias");
    m->q1_w = get("q_mlp.0.weight"); m->q1_b = get("q_mlp.0.bias");
    m->q2_w = get("q_mlp.2.weight"); m->q2_b = get("q_mlp.2.bias");
    m->s1_w = get("score_mlp.0.weight"); m->s1_b = get("score_mlp.0.bias");
    m->s2_w = get("score_mlp.2.weight"); m->s2_b = get("score_mlp.2.bias");
    m->v1_w = get("value_mlp.0.weight"); m->v1_b = get("value_mlp.0.bias");
    m->v2_w = get("value_mlp.2.weight"); m->v2_b = get("value_mlp.2.bias");
    PT_REQUIRE(m->v2_b, "model_bind: parameter table incomplete");
    if (m->dm.critic == 1) {
        m->op_w = get("oracle_proj.weight"); m->op_b = get("oracle_proj.bias");
        m->cread = get("critic_readout");
        bind_block(byname, "critic_blocks.0.", m->cblk);
        m->ov1_w = get("oracle_value_mlp.0.weight"); m->ov1_b = get("oracle_value_mlp.0.bias");
        m->ov2_w = get("oracle_value_mlp.2.weight"); m->ov2_b = get("oracle_value_mlp.2.bias");
        m->ah_w = get("aux_hand.weight"); m->ah_b = get("aux_hand.bias");
        m->ap_w = get("aux_prize.weight"); m->ap_b = get("aux_prize.bias");
        PT_REQUIRE(m->op_w && m->cblk.f2b && m->ap_b, "model_bind: parameter table incomplete");
    }
    return PTCG_OK;
}

// the static-table chain's batch-independent buffers
static size_t carve_tables(PtcgModel* m, char* base) {
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const long NC = d.n_cards, NA = d.n_attacks, NS = d.n_skills;
    Carver c{base};
    m->card_attacks = reinterpret_cast<int*>(c.take(NC * PT_K_ATT));
    m->card_skills = reinterpret_cast<int*>(c.take(NC * PT_K_SK));
    m->a_amax = reinterpret_cast<int*>(c.take(NC * d.d_a));
    m->s_amax = reinterpret_cast<int*>(c.take(NC * d.d_c));
    m->att_in = c.take(NA * x.att_in); m->att_lin = c.take(NA * d.d_a); m->att_tab = c.take(NA * d.d_a);
    m->sk_in = c.take(NS * x.sk_in); m->sk_lin = c.take(NS * d.d_c); m->sk_tab = c.take(NS * d.d_c);
    m->card_in = c.take(NC * x.card_in); m->c_mu = c.take(NC); m->c_rs = c.take(NC);
    m->card_ln = c.take(NC * x.card_in);
    m->card_h1 = c.take(NC * PT_CARD_H); m->card_g1 = c.take(NC * PT_CARD_H);
    m->card_vec = c.take(NC * d.d_c);
    m->d_card_vec = c.take(NC * d.d_c); m->d_att_tab = c.take(NA * d.d_a); m->d_sk_tab = c.take(NS * d.d_c);
    m->d_card_h = c.take(NC * PT_CARD_H);
    m->d_card_ln = c.take(NC * x.card_in); m->d_card_in = c.take(NC * x.card_in);
    m->d_att_lin = c.take(NA * d.d_a); m->d_sk_lin = c.take(NS * d.d_c);
    return c.off;
}

extern "C" int ptcg_model_set_static(PtcgModel* m, const float* card_static, const float* att_static,
                                     const float* card_text, const float* att_text, const float* skill_text,
                                     const int32_t* card_attacks, const int32_t* card_skills) {
    PT_REQUIRE(m, "model_set_static: null model");
    PT_REQUIRE(m->dm.tables == 1, "model_set_static: the model has learned tables (tables=0)");
    PT_REQUIRE(card_static && att_static && card_text && att_text && skill_text && card_attacks && card_skills,
               "model_set_static: null table");
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const long NC = d.n_cards, NA = d.n_attacks, NS = d.n_skills;
    for (long i = 0; i < NC * PT_K_ATT; ++i)
        PT_REQUIRE(card_attacks[i] >= 0 && card_attacks[i] < NA, "model_set_static: card_attacks[%ld]=%d "
                   "outside [0, %ld)", i, card_attacks[i], NA);
    for (long i = 0; i < NC * PT_K_SK; ++i)
        PT_REQUIRE(card_skills[i] >= 0 && card_skills[i] < NS, "model_set_static: card_skills[%ld]=%d "
                   "outside [0, %ld)", i, card_skills[i], NS);
    if (!m->tmem) {
        const size_t bytes = carve_tables(m, nullptr);
        PT_HIP(hipMalloc(&m->tmem, bytes));
        PT_HIP(hipMemset(m->tmem, 0, bytes));
        carve_tables(m, m->tmem);
    }
    auto put = [&](float* dst, long ld, int col0, const float* src, int w, long rows) -> int {
        PT_HIP(hipMemcpy2D(dst + col0, ld * sizeof(float), src, w * sizeof(float), w * sizeof(float), rows,
                           hipMemcpyHostToDevice));
        return PTCG_OK;
    };
    // concat inputs: [id | static | text] (the id columns are refreshed every forward)
    PT_TRY(put(m->att_in, x.att_in, PT_ID_A, att_static, PT_ATT_STATIC, NA));
    PT_TRY(put(m->att_in, x.att_in, PT_ID_A + PT_ATT_STATIC, att_text, PT_ATT_TEXT, NA));
    PT_TRY(put(m->sk_in, x.sk_in, PT_ID_A, skill_text, PT_SKILL_TEXT, NS));
    PT_TRY(put(m->card_in, x.card_in, PT_ID_C, card_static, PT_CARD_STATIC, NC));
    PT_TRY(put(m->card_in, x.card_in, PT_ID_C + PT_CARD_STATIC, card_text, PT_CARD_TEXT, NC));
    PT_HIP(hipMemcpy(m->card_attacks, card_attacks, NC * PT_K_ATT * sizeof(int), hipMemcpyHostToDevice));
    PT_HIP(hipMemcpy(m->card_skills, card_skills, NC * PT_K_SK * sizeof(int), hipMemcpyHostToDevice));
    m->card = m->card_vec;
    m->att = m->att_tab;
    m->dcard = m->d_card_vec;
    m->datt = m->d_att_tab;
    return PTCG_OK;
}

extern "C" int ptcg_model_set_precision(PtcgModel* m, int prec) {
    PT_REQUIRE(m && (prec == 0 || prec == 1), "model_set_precision: precision must be 0 (fp32) or 1 (bf16)");
    PT_REQUIRE(prec == 0 || (m->dm.d % 8 == 0 && m->dm.ffn % 8 == 0 && m->dm.d <= 256),
               "model_set_precision: bf16 activations need d and ffn multiples of 8 and d <= 256 (d=%d, ffn=%d)",
               m->dm.d, m->dm.ffn);
    m->prec = prec;
    return PTCG_OK;
}

extern "C" int ptcg_model_bind_returns(PtcgModel* m, const float* returns) {
    PT_REQUIRE(m, "model_bind_returns: null model");
    m->ret = returns;
    return PTCG_OK;
}

static void carve_block(Carver& c, BlockA& a, long NL, const PtcgDims& d) {
    const long D = d.d;
    a.ln1 = c.take(NL * D); a.mu1 = c.take(NL); a.rs1 = c.take(NL);
    a.qkv = c.take(NL * 3 * D); a.ctx = c.take(NL * D); a.lse = c.take(NL * d.heads);
    a.xmid = c.take(NL * D);
    a.ln2 = c.take(NL * D); a.mu2 = c.take(NL); a.rs2 = c.take(NL);
    a.ffp = c.take(NL * d.ffn); a.ffa = c.take(NL * d.ffn);
}

static void carve_bw(Carver& c, BlockW& w, const PtcgDims& d) {
    const long D = d.d, F = d.ffn;
    w.qkv = c.take_bf(3 * D * D); w.qkvT = c.take_bf(3 * D * D);
    w.proj = c.take_bf(D * D); w.projT = c.take_bf(D * D);
    w.f1 = c.take_bf(F * D); w.f1T = c.take_bf(F * D);
    w.f2 = c.take_bf(D * F); w.f2T = c.take_bf(D * F);
}

static size_t carve(PtcgModel* m, char* base) {
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const long N = m->N, Lt = d.l_tok, Ls = x.l_seq, NL = N * Ls, NO = d.n_opt, D = d.d;
    const bool crit = d.critic == 1, train = m->train;
    const long NLC = crit ? N * x.l_crit : 0, NLmax = NL > NLC ? NL : NLC, NK = N * x.n_orc;
    Carver c{base};
    const long tok_rows = m->compact ? NL : N * Lt;   // compact: token rows share the trunk row index
    m->tok_cat = c.take(tok_rows * x.tok_in);
    m->tokp = c.take(tok_rows * D);
    if (m->compact) {
        m->c_act = reinterpret_cast<int*>(c.take(NL));
        m->c_cnt = reinterpret_cast<int*>(c.take(N));
        m->c_off = reinterpret_cast<int*>(c.take(N + 1));
        m->c_map = reinterpret_cast<int*>(c.take(NL));
        m->c_rsam = reinterpret_cast<int*>(c.take(NL));
        m->c_rpos = reinterpret_cast<int*>(c.take(NL));
        m->rd_buf = c.take(N * D);
        m->Tr = m->c_off ? m->c_off + N : nullptr;
    } else {
        m->Tr = nullptr;
    }
    m->o_cnt = reinterpret_cast<int*>(c.take(N));
    m->o_off = reinterpret_cast<int*>(c.take(N + 1));
    m->o_row = reinterpret_cast<int*>(c.take(N * NO));
    m->glob_in = c.take(N * d.global_f);
    m->g1 = c.take(N * d.g); m->g1a = c.take(N * d.g);
    m->dec_in = c.take(N * x.dec_in);
    m->d1 = c.take(N * PT_DEC_H); m->d1a = c.take(N * PT_DEC_H);
    m->gd = c.take(N * x.bcast_in);
    m->bc = c.take(N * D);
    m->keep = c.take(NL);
    m->x.resize(train ? d.layers + 1 : 2);
    for (auto& p : m->x) p = c.take(NL * D);
    m->ba.resize(train ? d.layers : 1);
    for (auto& a : m->ba) carve_block(c, a, NL, d);
    m->h = c.take(NL * D); m->lnf_mu = c.take(NL); m->lnf_rs = c.take(NL);
    m->ocard = c.take(N * NO * d.d_c); m->oatt = c.take(N * NO * d.d_a);
    m->q_in = c.take(N * NO * x.q_in);
    m->q1 = c.take(N * NO * D); m->q1a = c.take(N * NO * D);
    m->sc_in = c.take(N * NO * x.score_in);
    m->s1 = c.take(N * NO * PT_SC_H); m->s1a = c.take(N * NO * PT_SC_H);
    m->val_in = c.take(N * x.val_in);
    m->v1 = c.take(N * PT_VAL_H); m->v1a = c.take(N * PT_VAL_H);
    m->out = c.take(N * (NO + 1));
    if (crit) {
        m->otok_in = c.take(NK * x.orc_in); m->otok = c.take(NK * D);
        m->ckeep = c.take(NLC);
        m->xc = c.take(NLC * D); m->xco = c.take(NLC * D);
        carve_block(c, m->cba, NLC, d);
        m->ov_in = c.take(N * x.val_in);
        m->ov1 = c.take(N * PT_VAL_H); m->ov1a = c.take(N * PT_VAL_H);
        if (train) {
            m->bv = c.take(N);
            m->hand_lin = c.take(N * d.n_cards);
            m->prize_all = c.take(NL);
            m->d_hand = c.take(N * d.n_cards); m->d_prize = c.take(NL); m->d_blind = c.take(N);
            m->dxc = c.take(NLC * D); m->dxc2 = c.take(NLC * D);
            m->dotok = c.take(NK * D); m->dotok_in = c.take(NK * x.orc_in);
            m->dov1 = c.take(N * PT_VAL_H); m->dovin = c.take(N * x.val_in);
            m->aux_cnt = reinterpret_cast<int*>(c.take(64));
        }
    }
    m->bw.resize(d.layers);
    for (auto& w : m->bw) carve_bw(c, w, d);
    if (crit) carve_bw(c, m->cbw, d);
    if (!train) {   // forward GEMMs use the workspace for balanced tail tiles only
        m->ws_floats = 4L << 20;
        m->ws = c.take(m->ws_floats);
        return c.off;
    }
    // backward scratch (block scratch sized for the longer of trunk and critic)
    m->dxa = c.take(NL * D); m->dxb = c.take(NL * D);
    m->dffn = c.take(NLmax * d.ffn); m->dln = c.take(NLmax * D);
    m->dqkv = c.take(NLmax * 3 * D); m->dctx = c.take(NLmax * D);
    m->dsc = c.take(N * NO * x.score_in); m->ds1 = c.take(N * NO * PT_SC_H);
    m->dq = c.take(N * NO * D); m->dq1 = c.take(N * NO * D);
    m->dqin = c.take(N * NO * x.q_in);
    m->docard = c.take(N * NO * d.d_c); m->doatt = c.take(N * NO * d.d_a);
    m->dvin = c.take(N * x.val_in); m->dv1 = c.take(N * PT_VAL_H);
    m->dgd = c.take(N * x.bcast_in); m->dd1 = c.take(N * PT_DEC_H); m->dg1 = c.take(N * d.g);
    m->ddec = c.take(N * x.dec_in);
    m->dtokp = c.take(tok_rows * D); m->dtokcat = c.take(tok_rows * x.tok_in);
    m->dbc = c.take(N * D);
    m->dAh = reinterpret_cast<float*>(c.take_bf(NLmax * D));
    m->dCh = reinterpret_cast<float*>(c.take_bf(NLmax * D));
    // table-scatter accumulators: the card, attack and skill tables plus the
    // small ones (zone, owner, option type, select type, context) of one site
    m->det.acc_len = (long)d.n_cards * d.d_c + (long)d.n_attacks * d.d_a + (long)d.n_skills * d.d_c + 4096;
    m->det.acc = reinterpret_cast<unsigned long long*>(c.take(2 * m->det.acc_len));
    m->det.part = c.take(DET_MAX_SRC * DET_PART);
    m->det.scale = reinterpret_cast<double*>(c.take(2 * DET_MAX_TAB));
    // workspace: split-K partials, column-sum / LayerNorm / head partials
    m->ws_floats = 16L << 20;
    long ln_part = 4096L * (D > x.card_in ? D : x.card_in);   // LayerNorm dW/dB partials (layernorm.hip)
    if (ln_part > m->ws_floats) m->ws_floats = ln_part;
    m->ws = c.take(m->ws_floats);
    m->ws2_floats = 16L << 20;   // the side stream's weight-gradient split-K partials
    m->ws2 = c.take(m->ws2_floats);
    // the trunk attention backward parks dS here (fp32 size covers both precisions)
    m->attn_ws_bytes = m->train ? pt_attn_bwd_ws_bytes(N, x.l_seq, d.heads, x.dh, 0) : 0;
    m->attn_ws = m->attn_ws_bytes ? c.take((m->attn_ws_bytes + 3) / 4) : nullptr;
    return c.off;
}

static int reg(PtcgModel* m, int n, bool train) {
    if (!m->rows_h) PT_HIP(hipHostMalloc((void**)&m->rows_h, 2 * sizeof(int), hipHostMallocDefault));
    if (m->mem) {
        PT_HIP(hipFree(m->mem));
        m->mem = nullptr;
    }
    m->N = n;
    m->train = train;
    m->compact = m->dm.critic == 0;
    m->det = DetCtx{};
    if (train && !m->wg_s) {
        PT_HIP(hipStreamCreateWithFlags(&m->wg_s, hipStreamNonBlocking));
        for (auto& e : m->wg_ev) PT_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    size_t bytes = carve(m, nullptr);
    PT_HIP(hipMalloc(&m->mem, bytes));
    m->mem_bytes = bytes;
    carve(m, m->mem);
    // the table-scatter accumulators start at zero (each site's finish re-zeroes them)
    if (m->det.acc) PT_HIP(hipMemset(m->det.acc, 0, m->det.acc_len * sizeof(unsigned long long)));
    return PTCG_OK;
}

extern "C" int ptcg_model_set_skip_masked_options(PtcgModel* m, int on) {
    PT_REQUIRE(m, "model_set_skip_masked_options: null model");
    m->skip_masked = on != 0;
    return PTCG_OK;
}

extern "C" int ptcg_model_set_sync_free(PtcgModel* m, int on) {
    PT_REQUIRE(m, "model_set_sync_free: null model");
    m->sync_free = on != 0;
    return PTCG_OK;
}

extern "C" int ptcg_model_reg_train(PtcgModel* m, int n) {
    PT_REQUIRE(m && n >= 2, "model_reg_train: need n >= 2 rows");
    return reg(m, n, true);
}

extern "C" int ptcg_model_reg_rollout(PtcgModel* m, int n) {
    PT_REQUIRE(m && n >= 1, "model_reg_rollout: need n >= 1 rows");
    return reg(m, n, false);
}

extern "C" void ptcg_model_free(PtcgModel* m) {
    if (!m) return;
    if (m->wg_s) {
        (void)hipStreamSynchronize(m->wg_s);
        for (auto e : m->wg_ev)
            if (e) (void)hipEventDestroy(e);
        (void)hipStreamDestroy(m->wg_s);
    }
    if (m->mem) (void)hipFree(m->mem);
    if (m->tmem) (void)hipFree(m->tmem);
    if (m->rows_h) (void)hipHostFree(m->rows_h);
    delete m;
}

size_t pt_model_act_bytes(const PtcgModel* m) { return m->mem_bytes; }
float* pt_model_out(const PtcgModel* m) { return m->out; }
float* pt_model_ws(const PtcgModel* m, long* floats) { *floats = m->ws_floats; return m->ws; }

// ------------------------------------------------------------ forward
// rows / Tr / coff of a compact layout: launch rows, device row count
// (nullable) and per-sample row offsets (rows 0, coff null: N * L rows)
// bw (bf16 variant): the block's bf16 weight copies; the block's activations
// are then stored in bf16 (the residual stream xin / xmid / xout stays fp32)
// fp32 blocks: ln1_done = the previous block's FFN2 launch already wrote this
// block's LayerNorm 1 (a.ln1, mu1, rs1); next (nullable) = the LayerNorm that
// reads xout (the next block's LayerNorm 1 or the trunk's final one), run with
// the FFN2 residual product
static int block_fwd(PtcgModel* m, const BlockP& w, const BlockA& a, int L, const float* keep, const float* xin,
                     float* xout, hipStream_t s, int rows = 0, const int* Tr = nullptr,
                     const int* coff = nullptr, const BlockW* bw = nullptr, bool ln1_done = false,
                     const LnOut* next = nullptr) {
    const PtcgDims& d = m->dm;
    const int NL = rows ? rows : m->N * L, D = d.d;
    if (bw) {
        if (!ln1_done) PT_TRY(pt_ln_fwd(xin, D, w.ln1w, w.ln1b, a.ln1, D, a.mu1, a.rs1, NL, D, s, Tr, 1));
        PT_TRY(blin(m, a.ln1, D, bw->qkv, w.qkvb, a.qkv, 3 * D, NL, EPI_BIAS, true, nullptr, nullptr, s, Tr));
        PT_TRY(pt_attn_fwd(a.qkv, keep, a.ctx, a.lse, m->N, L, d.heads, m->dx.dh, s, coff, 2));
        PT_TRY(blin_resid_ln(m, a.ctx, D, bw->proj, w.projb, a.xmid, D, NL, xin,
                             LnOut{w.ln2w, w.ln2b, a.ln2, a.mu2, a.rs2, 1}, s, Tr));
        PT_TRY(blin(m, a.ln2, D, bw->f1, w.f1b, a.ffp, d.ffn, NL, EPI_BIAS_GELU_D, true, nullptr, a.ffa, s, Tr));
        if (next) return blin_resid_ln(m, a.ffa, d.ffn, bw->f2, w.f2b, xout, D, NL, a.xmid, *next, s, Tr);
        PT_TRY(blin(m, a.ffa, d.ffn, bw->f2, w.f2b, xout, D, NL, EPI_BIAS_RESID, false, a.xmid, nullptr, s, Tr));
        return PTCG_OK;
    }
    if (!ln1_done) PT_TRY(pt_ln_fwd(xin, D, w.ln1w, w.ln1b, a.ln1, D, a.mu1, a.rs1, NL, D, s, Tr));
    PT_TRY(linf(m, a.ln1, w.qkvw, w.qkvb, a.qkv, NL, D, 3 * D, EPI_BIAS, nullptr, nullptr, s, Tr));
    PT_TRY(pt_attn_fwd(a.qkv, keep, a.ctx, a.lse, m->N, L, d.heads, m->dx.dh, s, coff, m->prec));
    PT_TRY(lin_resid_ln(m, a.ctx, w.projw, w.projb, a.xmid, NL, D, D, xin, LnOut{w.ln2w, w.ln2b, a.ln2, a.mu2, a.rs2},
                        s, Tr));
    PT_TRY(linf(m, a.ln2, w.f1w, w.f1b, a.ffp, NL, D, d.ffn, EPI_BIAS_GELU_D, nullptr, a.ffa, s, Tr));
    if (next) return lin_resid_ln(m, a.ffa, w.f2w, w.f2b, xout, NL, d.ffn, D, a.xmid, *next, s, Tr);
    PT_TRY(linf(m, a.ffa, w.f2w, w.f2b, xout, NL, d.ffn, D, EPI_BIAS_RESID, a.xmid, nullptr, s, Tr));
    return PTCG_OK;
}

// AttackVec, SkillVec, CardVec rebuilt from the static tables (tables_fwd,
// ptcg_model2.cu:422-452)
static int tables_fwd(PtcgModel* m, hipStream_t s) {
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const int NC = d.n_cards, NA = d.n_attacks, NS = d.n_skills, DA = d.d_a, DC = d.d_c;
    const int pa = PT_ID_C + PT_CARD_STATIC + PT_CARD_TEXT;   // first pool column of card_in
    PT_TRY(pt_copy_cols(m->att_in, x.att_in, m->aid_emb, PT_ID_A, NA, PT_ID_A, s));
    PT_TRY(lin(m, m->att_in, x.att_in, m->am_w, m->am_b, m->att_lin, DA, NA, x.att_in, DA, EPI_BIAS_GELU_D, nullptr, 0,
               m->att_tab, DA, s));
    PT_TRY(pt_copy_cols(m->sk_in, x.sk_in, m->sid_emb, PT_ID_A, NS, PT_ID_A, s));
    PT_TRY(lin(m, m->sk_in, x.sk_in, m->sm_w, m->sm_b, m->sk_lin, DC, NS, x.sk_in, DC, EPI_BIAS_GELU_D, nullptr, 0,
               m->sk_tab, DC, s));
    PT_TRY(pt_copy_cols(m->card_in, x.card_in, m->cid_emb, PT_ID_C, NC, PT_ID_C, s));
    PT_TRY(pt_pool_fwd(m->att_tab, DA, m->card_attacks, PT_K_ATT, NC, m->card_in, x.card_in, pa, pa + DA,
                       m->a_amax, s));
    PT_TRY(pt_pool_fwd(m->sk_tab, DC, m->card_skills, PT_K_SK, NC, m->card_in, x.card_in, pa + 2 * DA,
                       pa + 2 * DA + DC, m->s_amax, s));
    PT_TRY(pt_ln_fwd(m->card_in, x.card_in, m->cln_w, m->cln_b, m->card_ln, x.card_in, m->c_mu, m->c_rs, NC,
                     x.card_in, s));
    PT_TRY(lin(m, m->card_ln, x.card_in, m->c1_w, m->c1_b, m->card_h1, PT_CARD_H, NC, x.card_in, PT_CARD_H,
               EPI_BIAS_GELU_D, nullptr, 0, m->card_g1, PT_CARD_H, s));
    PT_TRY(linf(m, m->card_g1, m->c3_w, m->c3_b, m->card_vec, NC, PT_CARD_H, DC, EPI_BIAS, nullptr, nullptr, s));
    return PTCG_OK;
}

extern "C" int ptcg_model_forward(PtcgModel* m, const float* obs, const int32_t* row_idx, int n,
                                  float** out, void* stream) {
    PT_REQUIRE(m && obs && m->P, "model_forward: model not bound");
    PT_REQUIRE(m->mem, "model_forward: activations not registered (call ptcg_model_reg_train)");
    PT_REQUIRE(n == m->N, "model_forward: need exactly %d rows (activations are sized at "
               "registration, bindings.cu:227-233), got %d", m->N, n);
    PT_REQUIRE(m->dm.tables == 0 || m->tmem, "model_forward: static tables not uploaded (ptcg_model_set_static)");
    hipStream_t s = (hipStream_t)stream;
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const int N = m->N, Lt = d.l_tok, NO = d.n_opt, D = d.d, G = d.g;
    m->obs = obs;
    m->idx = row_idx;
    GatherCtx c{obs, row_idx, (long)m->off.size, N, d, x, m->off};
    const int* Tr = m->Tr;
    const int* coff = m->compact ? m->c_off : nullptr;
    m->rows = N * x.l_seq;
    m->Tdev = nullptr;
    m->orows = N * NO;
    m->Odev = nullptr;
    const bool skip = m->skip_masked;
    m->skip_fwd = skip;
    // The global / decision MLPs, the broadcast product and the option rows'
    // card / attack projections read only the observations and the tables:
    // in a training forward (no launch profile open) they run on the side
    // stream (workspace ws2) beside the row compaction, the token path and the
    // trunk, forked here (after the static-table chain, which feeds them), the
    // projections after the main stream's compaction (wg_ev[8]).  They join
    // where their outputs are read (bc: the trunk input; the projections: the
    // option rows' q_in).  Each fork and join is recorded before the main
    // stream's next launch is enqueued and taken after (see wg_mark).
    const bool fside = m->train && m->wg_s != nullptr && !pt_prof_active();
    hipStream_t sf = fside ? m->wg_s : s;
    float* fws = fside ? m->ws2 : m->ws;
    const long fwsn = fside ? m->ws2_floats : m->ws_floats;
    if (d.tables == 1) PT_TRY(tables_fwd(m, s));
    if (fside) PT_HIP(hipEventRecord(m->wg_ev[0], s));
    if (m->compact) {
        PT_TRY(pt_compact_map(c, m->c_act, m->c_cnt, m->c_off, m->c_map, m->c_rsam, m->c_rpos, s));
        c.coff = m->c_off; c.rowmap = m->c_map; c.rsam = m->c_rsam; c.rpos = m->c_rpos; c.rows = Tr;
    }
    if (skip) {
        PT_TRY(pt_opt_map(c, m->o_cnt, m->o_off, m->o_row, s));
        c.orow = m->o_row; c.ooff = m->o_off; c.orows = m->o_off + N;
    }
    if (fside) PT_HIP(hipStreamWaitEvent(m->wg_s, m->wg_ev[0], 0));
    // the per-sample MLPs and the broadcast product (one launch where the
    // widths allow: a chain of separate products is a dozen dependent
    // launches, whose latency set when the trunk could start)
    PT_TRY(pt_glob_in(c, m->glob_in, sf));
    PT_TRY(pt_dec_in_fwd(c, m->card, m->att, m->semb, m->cemb, m->dec_in, sf));
    const MlpChain mc{N, d.global_f, G, x.dec_in, PT_DEC_H, D, m->glob_in, m->dec_in,
                      m->g1_w, m->g1_b, m->g2_w, m->g2_b, m->d1_w, m->d1_b, m->d2_w, m->d2_b, m->bc_w, m->bc_b,
                      m->g1, m->g1a, m->d1, m->d1a, m->gd, m->bc};
    if (pt_mlp_chain_fits(mc)) {
        PT_TRY(pt_mlp_chain_fwd(mc, sf));
    } else {
        PT_TRY(lin_ws(m, fws, fwsn, m->glob_in, d.global_f, m->g1_w, m->g1_b, m->g1, G, N, d.global_f, G,
                      EPI_BIAS_GELU_D, nullptr, G, m->g1a, G, sf));
        PT_TRY(lin_ws(m, fws, fwsn, m->g1a, G, m->g2_w, m->g2_b, m->gd, x.bcast_in, N, G, G, EPI_BIAS, nullptr, 0,
                      nullptr, 0, sf));
        PT_TRY(lin_ws(m, fws, fwsn, m->dec_in, x.dec_in, m->d1_w, m->d1_b, m->d1, PT_DEC_H, N, x.dec_in, PT_DEC_H,
                      EPI_BIAS_GELU_D, nullptr, PT_DEC_H, m->d1a, PT_DEC_H, sf));
        PT_TRY(lin_ws(m, fws, fwsn, m->d1a, PT_DEC_H, m->d2_w, m->d2_b, m->gd + G, x.bcast_in, N, PT_DEC_H,
                      PT_DEC_H, EPI_BIAS, nullptr, 0, nullptr, 0, sf));
        PT_TRY(lin_ws(m, fws, fwsn, m->gd, x.bcast_in, m->bc_w, m->bc_b, m->bc, D, N, x.bcast_in, D, EPI_BIAS,
                      nullptr, 0, nullptr, 0, sf));
    }
    if (fside) PT_HIP(hipEventRecord(m->wg_ev[6], m->wg_s));
    if (m->compact || skip) {
        if (m->sync_free) {
            m->Tdev = m->compact ? Tr : nullptr;
            m->Odev = skip ? m->o_off + N : nullptr;
        } else {
            // the step's one host read-back: the trunk and option row counts
            // size every launch that follows
            if (m->compact) PT_HIP(hipMemcpyAsync(m->rows_h, Tr, sizeof(int), hipMemcpyDeviceToHost, s));
            if (skip) PT_HIP(hipMemcpyAsync(m->rows_h + 1, m->o_off + N, sizeof(int), hipMemcpyDeviceToHost, s));
            PT_HIP(hipStreamSynchronize(s));
            if (m->compact) m->rows = m->rows_h[0];
            if (skip) m->orows = m->rows_h[1];
            PT_REQUIRE(m->rows >= N && m->rows <= N * x.l_seq, "model_forward: compact row count %d out of range",
                       m->rows);
            PT_REQUIRE(m->orows >= N && m->orows <= N * NO, "model_forward: option row count %d out of range",
                       m->orows);
        }
    }
    const int* Td = m->Tdev;
    const int tok_rows = m->compact ? m->rows : N * Lt;
    const int NJ = m->orows;
    const int* Od = m->Odev;
    const int oc0 = PT_TYPE_E + 2 * D, oa0 = oc0 + PT_OPT_E;
    if (fside) PT_HIP(hipEventRecord(m->wg_ev[8], s));   // the row maps are written
    PT_TRY(pt_tok_cat_fwd(c, m->card, m->zemb, m->oemb, m->tok_cat, s, tok_rows));
    PT_TRY(linf(m, m->tok_cat, m->tp_w, m->tp_b, m->tokp, tok_rows, x.tok_in, D, EPI_BIAS, nullptr, nullptr, s, Td));
    if (fside) PT_HIP(hipStreamWaitEvent(s, m->wg_ev[6], 0));   // bc for the trunk input
    const bool tr = m->train;
    const bool b16 = m->prec == 1;
    // at d = 256 the first block's LayerNorm 1 runs inside the trunk-input assembly
    const bool ln0 = D == 256;
    const BlockA& a0 = m->ba[0];
    if (ln0)
        PT_TRY(pt_x0_fwd(c, m->tokp, m->bc, m->readout, m->x[0], m->keep, s, m->blk[0].ln1w, m->blk[0].ln1b,
                         a0.ln1, a0.mu1, a0.rs1, b16 ? 1 : 0));
    else
        PT_TRY(pt_x0_fwd(c, m->tokp, m->bc, m->readout, m->x[0], m->keep, s));
    // the option rows' card / attack projections, captured after the trunk
    // input so that a replay's wait for bc does not wait for them as well
    if (fside) PT_HIP(hipStreamWaitEvent(m->wg_s, m->wg_ev[8], 0));   // option row map
    PT_TRY(pt_opt_gather_fwd(c, m->card, m->att, m->ocard, m->oatt, sf));
    PT_TRY(lin_ws(m, fws, fwsn, m->ocard, d.d_c, m->oc_w, m->oc_b, m->q_in + oc0, x.q_in, NJ, d.d_c, PT_OPT_E,
                  EPI_BIAS, nullptr, 0, nullptr, 0, sf, Od));
    PT_TRY(lin_ws(m, fws, fwsn, m->oatt, d.d_a, m->oa_w, m->oa_b, m->q_in + oa0, x.q_in, NJ, d.d_a, PT_OPT_E,
                  EPI_BIAS, nullptr, 0, nullptr, 0, sf, Od));
    if (fside) PT_HIP(hipEventRecord(m->wg_ev[7], m->wg_s));
    if (b16) PT_TRY(bf16_refresh(m, s));
    // each block's FFN2 residual product also runs the LayerNorm that reads
    // its output: the next block's LayerNorm 1 (bf16 output in the
    // mixed-precision blocks) or the final one (fp32)
    for (int i = 0; i < d.layers; ++i) {
        LnOut nx{m->lnf_w, m->lnf_b, m->h, m->lnf_mu, m->lnf_rs, 0};
        if (i + 1 < d.layers) {
            const BlockP& wn = m->blk[i + 1];
            const BlockA& an = m->ba[tr ? i + 1 : 0];
            nx = LnOut{wn.ln1w, wn.ln1b, an.ln1, an.mu1, an.rs1, b16 ? 1 : 0};
        }
        PT_TRY(block_fwd(m, m->blk[i], m->ba[tr ? i : 0], x.l_seq, m->keep, m->x[tr ? i : i % 2],
                         m->x[tr ? i + 1 : (i + 1) % 2], s, m->rows, Td, coff, b16 ? &m->bw[i] : nullptr,
                         i > 0 || ln0, &nx));
    }
    const int NL = N * x.l_seq;

    // option scorer over the option rows (all N * n_opt, or the legal ones);
    // their card / attack projections ran above (side stream: joined here)
    if (fside) PT_HIP(hipStreamWaitEvent(s, m->wg_ev[7], 0));
    PT_TRY(pt_q_in_fwd(c, m->h, m->temb, m->q_in, s));
    PT_TRY(linf(m, m->q_in, m->q1_w, m->q1_b, m->q1, NJ, x.q_in, D, EPI_BIAS_GELU_D, nullptr, m->q1a, s, Od));
    PT_TRY(lin(m, m->q1a, D, m->q2_w, m->q2_b, m->sc_in, x.score_in, NJ, D, D, EPI_BIAS, nullptr, 0, nullptr, 0, s,
               Od));
    PT_TRY(pt_sc_in_fwd(c, m->h, m->gd, m->sc_in, s));
    PT_TRY(linf(m, m->sc_in, m->s1_w, m->s1_b, m->s1, NJ, x.score_in, PT_SC_H, EPI_BIAS_GELU_D, nullptr, m->s1a, s,
                Od));
    if (skip) PT_TRY(pt_fill_zero(m->out, (long)N * (NO + 1), s));   // masked slots read 0
    PT_TRY(pt_head_dot(m->s1a, NJ, PT_SC_H, m->s2_w, m->s2_b, m->out, NO, NO + 1, 0, s, skip ? m->o_row : nullptr, Od));
    // blind value head: the output value, or (oracle critic) an aux head
    PT_TRY(pt_val_in_fwd(c, m->h, m->gd, m->val_in, s));
    PT_TRY(linf(m, m->val_in, m->v1_w, m->v1_b, m->v1, N, x.val_in, PT_VAL_H, EPI_BIAS_GELU_D, nullptr, m->v1a, s));
    if (d.critic == 0) {
        PT_TRY(pt_head_dot(m->v1a, N, PT_VAL_H, m->v2_w, m->v2_b, m->out, 1, NO + 1, NO, s));
    } else {
        if (tr) {   // training only (ptcg_model3.cu:353-363): blind value and belief heads
            PT_TRY(pt_head_dot(m->v1a, N, PT_VAL_H, m->v2_w, m->v2_b, m->bv, 1, 1, 0, s));
            PT_TRY(linf(m, m->val_in, m->ah_w, m->ah_b, m->hand_lin, N, x.val_in, d.n_cards, EPI_BIAS, nullptr,
                        nullptr, s));
            PT_TRY(pt_head_dot(m->h, NL, D, m->ap_w, m->ap_b, m->prize_all, 1, 1, 0, s));
        }
        // oracle critic top (ptcg_model3.cu:334-351)
        const int NK = N * x.n_orc;
        PT_TRY(pt_otok_in(c, m->card, m->keep, m->otok_in, m->ckeep, s));
        PT_TRY(linf(m, m->otok_in, m->op_w, m->op_b, m->otok, NK, x.orc_in, D, EPI_BIAS, nullptr, nullptr, s));
        PT_TRY(pt_xc_fwd(m->cread, m->h, m->otok, m->xc, N, x.l_seq, x.n_orc, D, s));
        PT_TRY(block_fwd(m, m->cblk, m->cba, x.l_crit, m->ckeep, m->xc, m->xco, s, 0, nullptr, nullptr,
                         b16 ? &m->cbw : nullptr));
        PT_TRY(pt_val_in_fwd(c, m->xco, m->gd, m->ov_in, s, x.l_crit));
        PT_TRY(linf(m, m->ov_in, m->ov1_w, m->ov1_b, m->ov1, N, x.val_in, PT_VAL_H, EPI_BIAS_GELU_D, nullptr, m->ov1a, s));
        PT_TRY(pt_head_dot(m->ov1a, N, PT_VAL_H, m->ov2_w, m->ov2_b, m->out, 1, NO + 1, NO, s));
    }
    if (out) *out = m->out;
    // stage dumps for parity bisection (the reference's PTCG_DUMP_DIR,
    // ptcg_model3.cu:371-400); never inside a capture
    const char* dump_dir = getenv("PTCG_DUMP_DIR");
    if (dump_dir && dump_dir[0]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        PT_HIP(hipStreamIsCapturing(s, &cs));
        if (cs == hipStreamCaptureStatusNone) PT_TRY(ptcg_model_dump_stages(m, dump_dir, s));
    }
    return PTCG_OK;
}

// Every named stage of the last forward as raw fp32 files <dir>/<name>.bin
// in the full layout the reference dumps (ptcg_model3.cu:222-231,371-400):
// per-sample stages (N, ...), token stages (N, l_tok, ...), trunk stages
// (N, l_seq, d), option stages (N, n_opt, ...).  Rows the compact trunk or
// the masked-option skip did not compute are written as 0.  Debug only:
// synchronises the stream and copies through the host.
extern "C" int ptcg_model_dump_stages(PtcgModel* m, const char* dir, void* stream) {
    PT_REQUIRE(m && dir && m->obs, "model_dump_stages: run a forward first");
    hipStream_t s = (hipStream_t)stream;
    PT_HIP(hipStreamSynchronize(s));
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const long N = m->N, Lt = d.l_tok, Ls = x.l_seq, NO = d.n_opt, D = d.d;
    auto d2h = [&](const void* src, long n, std::vector<float>& out) -> int {
        out.resize(n);
        if (n) PT_HIP(hipMemcpy(out.data(), src, n * sizeof(float), hipMemcpyDeviceToHost));
        return PTCG_OK;
    };
    auto write = [&](const char* name, const std::vector<float>& v) -> int {
        const std::string path = std::string(dir) + "/" + name + ".bin";
        FILE* f = fopen(path.c_str(), "wb");
        PT_REQUIRE(f, "model_dump_stages: cannot open %s", path.c_str());
        const size_t w = fwrite(v.data(), sizeof(float), v.size(), f);
        fclose(f);
        PT_REQUIRE(w == v.size(), "model_dump_stages: short write to %s", path.c_str());
        return PTCG_OK;
    };
    // columns [c0, c0 + w) of n rows of leading dimension ld
    auto cols = [&](const char* name, const float* src, long n, long ld, long c0, long w) -> int {
        std::vector<float> a, o((size_t)n * w);
        PT_TRY(d2h(src, n * ld, a));
        for (long r = 0; r < n; ++r)
            for (long k = 0; k < w; ++k) o[r * w + k] = a[r * ld + c0 + k];
        return write(name, o);
    };
    // compact trunk rows: row r holds (sample rsam[r], position rpos[r])
    int rows = (int)(N * Ls);
    std::vector<int> rsam, rpos;
    if (m->compact) {
        PT_HIP(hipMemcpy(&rows, m->Tr, sizeof(int), hipMemcpyDeviceToHost));
        PT_REQUIRE(rows >= 0 && rows <= N * Ls, "model_dump_stages: row count %d", rows);
        rsam.resize(rows);
        rpos.resize(rows);
        if (rows) {
            PT_HIP(hipMemcpy(rsam.data(), m->c_rsam, rows * sizeof(int), hipMemcpyDeviceToHost));
            PT_HIP(hipMemcpy(rpos.data(), m->c_rpos, rows * sizeof(int), hipMemcpyDeviceToHost));
        }
    }
    // a trunk-row buffer (tokens: pos_off = 1 drops READOUT) to (N, L, w)
    auto trunk = [&](const char* name, const float* src, long w, long L, int pos_off) -> int {
        std::vector<float> a, o((size_t)N * L * w, 0.f);
        const long nr = m->compact ? rows : N * L;
        PT_TRY(d2h(src, nr * w, a));
        for (long r = 0; r < nr; ++r) {
            const long n = m->compact ? rsam[r] : r / L;
            const long p = m->compact ? rpos[r] - pos_off : r % L;
            if (n < 0 || n >= N || p < 0 || p >= L) continue;
            std::copy(a.begin() + r * w, a.begin() + (r + 1) * w, o.begin() + (n * L + p) * w);
        }
        return write(name, o);
    };
    // option rows (all N * n_opt, or the legal ones through o_row) to (N, n_opt, w)
    int orows = (int)(N * NO);
    std::vector<int> orow;
    if (m->skip_fwd) {
        PT_HIP(hipMemcpy(&orows, m->o_off + N, sizeof(int), hipMemcpyDeviceToHost));
        PT_REQUIRE(orows >= 0 && orows <= N * NO, "model_dump_stages: option row count %d", orows);
        orow.resize(orows);
        if (orows) PT_HIP(hipMemcpy(orow.data(), m->o_row, orows * sizeof(int), hipMemcpyDeviceToHost));
    }
    auto opts = [&](const char* name, const float* src, long ld, long c0, long w) -> int {
        std::vector<float> a, o((size_t)N * NO * w, 0.f);
        PT_TRY(d2h(src, (long)orows * ld, a));
        for (long j = 0; j < orows; ++j) {
            const long dst = m->skip_fwd ? orow[j] : j;
            if (dst < 0 || dst >= N * NO) continue;
            for (long k = 0; k < w; ++k) o[dst * w + k] = a[j * ld + c0 + k];
        }
        return write(name, o);
    };
    PT_TRY(cols("card_vec", m->card, d.n_cards, d.d_c, 0, d.d_c));
    PT_TRY(cols("att_tab", m->att, d.n_attacks, d.d_a, 0, d.d_a));
    const int tok_pos_off = m->compact ? 1 : 0;
    PT_TRY(trunk("tok_cat", m->tok_cat, x.tok_in, Lt, tok_pos_off));
    PT_TRY(trunk("tokp", m->tokp, D, Lt, tok_pos_off));
    PT_TRY(cols("dec_in", m->dec_in, N, x.dec_in, 0, x.dec_in));
    PT_TRY(cols("g_out", m->gd, N, x.bcast_in, 0, d.g));
    PT_TRY(cols("d_out", m->gd, N, x.bcast_in, d.g, x.bcast_in - d.g));
    PT_TRY(cols("bc_out", m->bc, N, D, 0, D));
    PT_TRY(trunk("keep", m->keep, 1, Ls, 0));
    PT_TRY(trunk("x0", m->x[0], D, Ls, 0));
    if (m->train)
        for (int i = 1; i <= d.layers; ++i) {
            const std::string nm = "x" + std::to_string(i);
            PT_TRY(trunk(nm.c_str(), m->x[i], D, Ls, 0));
        }
    PT_TRY(trunk("h", m->h, D, Ls, 0));
    PT_TRY(opts("q_in", m->q_in, x.q_in, 0, x.q_in));
    PT_TRY(opts("q_vec", m->sc_in, x.score_in, 0, D));
    PT_TRY(opts("sc_in", m->sc_in, x.score_in, 0, x.score_in));
    PT_TRY(cols("out", m->out, N, NO + 1, 0, NO + 1));
    return PTCG_OK;
}

// ------------------------------------------------------------ backward
// dA holds d(x_out) on entry and d(x_in) on exit; dC is scratch for d(x_mid)
// bw (bf16 variant): m->dAh holds dA in bf16 on entry and holds the new dA in
// bf16 on exit (m->dCh likewise for dC)
static int block_bwd(PtcgModel* m, const BlockP& w, const BlockA& a, int L, const float* keep, const float* xin,
                     float* dA, float* dC, hipStream_t s, int rows = 0, const int* Tr = nullptr,
                     const int* coff = nullptr, const BlockW* bw = nullptr) {
    const PtcgDims& d = m->dm;
    const int NL = rows ? rows : m->N * L, D = d.d;
    // Weight gradients on the side stream (m->wg_s), each forked once its dY
    // is written; the main stream waits for the side stream only before it
    // overwrites a buffer a pending weight gradient reads: dffn (the previous
    // block's FFN1 dW), dC (its out-projection dW), dqkv (its QKV dW) and dA
    // (this block's FFN2 dW).
    hipStream_t s2 = m->wg_serial ? s : m->wg_s;
    // each weight gradient: marked where its dY is complete, taken after the
    // main stream's next product (see wg_mark)
    if (bw) {
        PT_TRY(wg_mark(m, s));
        PT_TRY(wg_after(m, 2, s));
        PT_TRY(blin(m, m->dAh, D, bw->f2T, nullptr, m->dffn, d.ffn, NL, EPI_MUL, true, a.ffp, nullptr, s, Tr));
        PT_TRY(wg_take(m));
        PT_TRY(bldw(m, m->dAh, D, a.ffa, d.ffn, m->G(w.f2w), m->G(w.f2b), NL, s2, Tr));
        PT_TRY(wg_done(m, 1));
        PT_TRY(wg_mark(m, s));
        PT_TRY(wg_after(m, 3, s));   // dC (the LayerNorm's dx) is read by the previous block's dW
        PT_TRY(blin_dx_lnbwd(m, m->dffn, d.ffn, bw->f1T, NL, a.xmid, w.ln2w, a.mu2, a.rs2, dA, dC, m->G(w.ln2w),
                             m->G(w.ln2b), m->dCh, s, Tr));
        PT_TRY(wg_take(m));
        PT_TRY(bldw(m, m->dffn, d.ffn, a.ln2, D, m->G(w.f1w), m->G(w.f1b), NL, s2, Tr));
        PT_TRY(wg_done(m, 2));
        PT_TRY(wg_mark(m, s));
        PT_TRY(blin(m, m->dCh, D, bw->projT, nullptr, m->dctx, D, NL, EPI_STORE, true, nullptr, nullptr, s, Tr));
        PT_TRY(wg_take(m));
        PT_TRY(bldw(m, m->dCh, D, a.ctx, D, m->G(w.projw), m->G(w.projb), NL, s2, Tr));
        PT_TRY(wg_done(m, 3));
        PT_TRY(wg_after(m, 4, s));
        PT_TRY(pt_attn_bwd(a.qkv, keep, a.ctx, a.lse, m->dctx, m->dqkv, m->N, L, d.heads, m->dx.dh, s, coff, 2,
                           m->attn_ws, m->attn_ws_bytes));
        PT_TRY(wg_mark(m, s));
        PT_TRY(wg_after(m, 1, s));   // dA and dAh are read by this block's FFN2 dW
        PT_TRY(blin_dx_lnbwd(m, m->dqkv, 3 * D, bw->qkvT, NL, xin, w.ln1w, a.mu1, a.rs1, dC, dA, m->G(w.ln1w),
                             m->G(w.ln1b), m->dAh, s, Tr));
        PT_TRY(wg_take(m));
        PT_TRY(bldw(m, m->dqkv, 3 * D, a.ln1, D, m->G(w.qkvw), m->G(w.qkvb), NL, s2, Tr));
        PT_TRY(wg_done(m, 4));
        return PTCG_OK;
    }
    PT_TRY(wg_mark(m, s));
    PT_TRY(wg_after(m, 2, s));
    PT_TRY(ldx_(m, dA, D, w.f2w, m->dffn, d.ffn, NL, d.ffn, D, EPI_MUL, a.ffp, d.ffn, s, Tr));
    PT_TRY(wg_take(m));
    PT_TRY(ldw_(m, dA, D, a.ffa, d.ffn, m->G(w.f2w), m->G(w.f2b), NL, d.ffn, D, s2, Tr, true));
    PT_TRY(wg_done(m, 1));
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, m->dffn, d.ffn, w.f1w, m->dln, D, NL, D, d.ffn, EPI_STORE, nullptr, 0, s, Tr));
    PT_TRY(wg_take(m));
    PT_TRY(ldw_(m, m->dffn, d.ffn, a.ln2, D, m->G(w.f1w), m->G(w.f1b), NL, D, d.ffn, s2, Tr, true));
    PT_TRY(wg_done(m, 2));
    PT_TRY(wg_after(m, 3, s));
    PT_TRY(pt_ln_bwd(m->dln, D, a.xmid, D, w.ln2w, a.mu2, a.rs2, dA, D, dC, D, m->G(w.ln2w),
                     m->G(w.ln2b), NL, D, m->ws, m->ws_floats, s, Tr));
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, dC, D, w.projw, m->dctx, D, NL, D, D, EPI_STORE, nullptr, 0, s, Tr));
    PT_TRY(wg_take(m));
    PT_TRY(ldw_(m, dC, D, a.ctx, D, m->G(w.projw), m->G(w.projb), NL, D, D, s2, Tr, true));
    PT_TRY(wg_done(m, 3));
    PT_TRY(wg_after(m, 4, s));
    PT_TRY(pt_attn_bwd(a.qkv, keep, a.ctx, a.lse, m->dctx, m->dqkv, m->N, L, d.heads, m->dx.dh, s, coff, m->prec,
                       m->attn_ws, m->attn_ws_bytes));
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, m->dqkv, 3 * D, w.qkvw, m->dln, D, NL, D, 3 * D, EPI_STORE, nullptr, 0, s, Tr));
    PT_TRY(wg_take(m));
    PT_TRY(ldw_(m, m->dqkv, 3 * D, a.ln1, D, m->G(w.qkvw), m->G(w.qkvb), NL, D, 3 * D, s2, Tr, true));
    PT_TRY(wg_done(m, 4));
    PT_TRY(wg_after(m, 1, s));
    PT_TRY(pt_ln_bwd(m->dln, D, xin, D, w.ln1w, a.mu1, a.rs1, dC, D, dA, D, m->G(w.ln1w),
                     m->G(w.ln1b), NL, D, m->ws, m->ws_floats, s, Tr));
    return PTCG_OK;
}

// the static-table chain from d CardVec / d AttackVec down to the id
// embeddings (tables_bwd, ptcg_model2.cu:454-485)
static int tables_bwd(PtcgModel* m, hipStream_t s) {
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const int NC = d.n_cards, NA = d.n_attacks, NS = d.n_skills, DA = d.d_a, DC = d.d_c;
    const int pa = PT_ID_C + PT_CARD_STATIC + PT_CARD_TEXT;
    PT_TRY(ldw_(m, m->d_card_vec, DC, m->card_g1, PT_CARD_H, m->G(m->c3_w), m->G(m->c3_b), NC, PT_CARD_H, DC, s));
    PT_TRY(ldx_(m, m->d_card_vec, DC, m->c3_w, m->d_card_h, PT_CARD_H, NC, PT_CARD_H, DC, EPI_MUL, m->card_h1,
                PT_CARD_H, s));
    PT_TRY(ldw_(m, m->d_card_h, PT_CARD_H, m->card_ln, x.card_in, m->G(m->c1_w), m->G(m->c1_b), NC, x.card_in,
                PT_CARD_H, s));
    PT_TRY(ldx_(m, m->d_card_h, PT_CARD_H, m->c1_w, m->d_card_ln, x.card_in, NC, x.card_in, PT_CARD_H, EPI_STORE,
                nullptr, 0, s));
    PT_TRY(pt_ln_bwd(m->d_card_ln, x.card_in, m->card_in, x.card_in, m->cln_w, m->c_mu, m->c_rs, nullptr, 0,
                     m->d_card_in, x.card_in, m->G(m->cln_w), m->G(m->cln_b), NC, x.card_in, m->ws, m->ws_floats, s));
    PT_TRY(pt_copy_cols(m->G(m->cid_emb), PT_ID_C, m->d_card_in, x.card_in, NC, PT_ID_C, s));
    // pool backward into the attack and skill tables (each (card, slot) adds mean + max parts)
    DetSite P;
    const int ta = P.add_table(m->d_att_tab, (long)NA * DA, 0, 2.0 * NC * PT_K_ATT);
    const int tk = P.add_table(m->d_sk_tab, (long)NS * DC, (long)NA * DA, 2.0 * NC * PT_K_SK);
    P.add_source(ta, m->d_card_in, x.card_in, pa, 2 * DA, NC);
    P.add_source(tk, m->d_card_in, x.card_in, pa + 2 * DA, 2 * DC, NC);
    PT_TRY(pt_det_prepare(m->det, P, s));
    PT_TRY(pt_pool_bwd(m->d_card_in, x.card_in, pa, pa + DA, m->a_amax, m->card_attacks, PT_K_ATT, NC, DA,
                       pt_det_sink(m->det, P, ta, DA), s));
    PT_TRY(pt_pool_bwd(m->d_card_in, x.card_in, pa + 2 * DA, pa + 2 * DA + DC, m->s_amax, m->card_skills, PT_K_SK,
                       NC, DC, pt_det_sink(m->det, P, tk, DC), s));
    PT_TRY(pt_det_finish(m->det, P, s));
    PT_TRY(pt_mul(m->d_att_tab, m->att_lin, m->d_att_lin, (long)NA * DA, s));
    PT_TRY(ldw_(m, m->d_att_lin, DA, m->att_in, x.att_in, m->G(m->am_w), m->G(m->am_b), NA, x.att_in, DA, s));
    PT_TRY(ldxw_(m, m->d_att_lin, DA, m->am_w, x.att_in, m->G(m->aid_emb), PT_ID_A, NA, PT_ID_A, DA, EPI_STORE,
                 nullptr, 0, s));
    PT_TRY(pt_mul(m->d_sk_tab, m->sk_lin, m->d_sk_lin, (long)NS * DC, s));
    PT_TRY(ldw_(m, m->d_sk_lin, DC, m->sk_in, x.sk_in, m->G(m->sm_w), m->G(m->sm_b), NS, x.sk_in, DC, s));
    PT_TRY(ldxw_(m, m->d_sk_lin, DC, m->sm_w, x.sk_in, m->G(m->sid_emb), PT_ID_A, NS, PT_ID_A, DC, EPI_STORE,
                 nullptr, 0, s));
    return PTCG_OK;
}

// oracle critic top + blind value + belief heads: the PPO value gradient
// (grad[:, NO]) enters at the oracle value; the aux losses at the heads
// (ptcg_model4.cu:26-101).  Adds into dxa (d h), dgd and dcard.
static int critic_bwd(PtcgModel* m, const GatherCtx& c, const float* grad, hipStream_t s) {
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const int N = m->N, NO = d.n_opt, D = d.d, NL = N * x.l_seq, NK = N * x.n_orc;
    PT_TRY(pt_aux_grads(c, m->hand_lin, m->prize_all, m->bv, m->ret, m->aux_cnt, m->d_hand, m->d_prize,
                        m->d_blind, s));
    // blind value (aux): d_blind -> value_mlp -> d [r | g]
    PT_TRY(pt_head_dot_dw(m->d_blind, 1, 1, 0, m->v1a, N, PT_VAL_H, m->G(m->v2_w), m->G(m->v2_b), m->ws,
                          m->ws_floats, s));
    PT_TRY(pt_head_dot_bwd(m->d_blind, 1, 1, 0, m->v2_w, m->v1, m->dv1, N, PT_VAL_H, s));
    PT_TRY(ldw_(m, m->dv1, PT_VAL_H, m->val_in, x.val_in, m->G(m->v1_w), m->G(m->v1_b), N, x.val_in, PT_VAL_H, s));
    PT_TRY(ldx_(m, m->dv1, PT_VAL_H, m->v1_w, m->dvin, x.val_in, N, x.val_in, PT_VAL_H, EPI_STORE, nullptr, 0, s));
    // opp-hand counts (shares the [r | g] input)
    PT_TRY(ldw_(m, m->d_hand, d.n_cards, m->val_in, x.val_in, m->G(m->ah_w), m->G(m->ah_b), N, x.val_in,
                d.n_cards, s));
    PT_TRY(ldx_(m, m->d_hand, d.n_cards, m->ah_w, m->dvin, x.val_in, N, x.val_in, d.n_cards, EPI_ACCUM, nullptr, 0, s));
    PT_TRY(pt_val_in_bwd(c, m->dvin, m->dxa, m->dgd, s));
    // prize head over the trunk output rows
    PT_TRY(pt_head_dot_dw(m->d_prize, 1, 1, 0, m->h, NL, D, m->G(m->ap_w), m->G(m->ap_b), m->ws, m->ws_floats, s));
    PT_TRY(pt_rank1_add(m->d_prize, m->ap_w, m->dxa, NL, D, s));
    // oracle value -> critic block -> h / oracle tokens / critic readout
    PT_TRY(pt_head_dot_dw(grad, 1, NO + 1, NO, m->ov1a, N, PT_VAL_H, m->G(m->ov2_w), m->G(m->ov2_b), m->ws,
                          m->ws_floats, s));
    PT_TRY(pt_head_dot_bwd(grad, 1, NO + 1, NO, m->ov2_w, m->ov1, m->dov1, N, PT_VAL_H, s));
    PT_TRY(ldw_(m, m->dov1, PT_VAL_H, m->ov_in, x.val_in, m->G(m->ov1_w), m->G(m->ov1_b), N, x.val_in, PT_VAL_H, s));
    PT_TRY(ldx_(m, m->dov1, PT_VAL_H, m->ov1_w, m->dovin, x.val_in, N, x.val_in, PT_VAL_H, EPI_STORE, nullptr, 0, s));
    PT_TRY(pt_fill_zero(m->dxc, (long)N * x.l_crit * D, s));
    PT_TRY(pt_val_in_bwd(c, m->dovin, m->dxc, m->dgd, s, x.l_crit));
    const bool b16 = m->prec == 1;
    if (b16) PT_TRY(pt_to_bf16(m->dxc, m->dAh, (long)N * x.l_crit * D, s));
    PT_TRY(block_bwd(m, m->cblk, m->cba, x.l_crit, m->ckeep, m->xc, m->dxc, m->dxc2, s, 0, nullptr, nullptr,
                     b16 ? &m->cbw : nullptr));
    PT_TRY(wg_after(m, 4, s));   // the critic block's weight gradients are done
    PT_TRY(pt_colsum(m->dxc, (long)x.l_crit * D, N, D, m->G(m->cread), m->ws, m->ws_floats, s));
    PT_TRY(pt_xc_bwd(m->dxc, m->dxa, m->dotok, N, x.l_seq, x.n_orc, D, s));
    PT_TRY(ldw_(m, m->dotok, D, m->otok_in, x.orc_in, m->G(m->op_w), m->G(m->op_b), NK, x.orc_in, D, s));
    PT_TRY(ldx_(m, m->dotok, D, m->op_w, m->dotok_in, x.orc_in, NK, x.orc_in, D, EPI_STORE, nullptr, 0, s));
    DetSite O;
    const int tc = O.add_table(m->dcard, (long)d.n_cards * d.d_c, 0, (double)NK);
    O.add_source(tc, m->dotok_in, x.orc_in, 0, d.d_c, NK);
    PT_TRY(pt_det_prepare(m->det, O, s));
    PT_TRY(pt_otok_bwd(c, m->dotok_in, pt_det_sink(m->det, O, tc, d.d_c), s));
    PT_TRY(pt_det_finish(m->det, O, s));
    return PTCG_OK;
}

extern "C" int ptcg_model_backward(PtcgModel* m, const float* grad, void* stream) {
    PT_REQUIRE(m && grad && m->mem && m->obs, "model_backward: run a forward first");
    PT_REQUIRE(m->train, "model_backward: activations were registered for rollout (ptcg_model_reg_train)");
    hipStream_t s = (hipStream_t)stream;
    for (bool& r : m->wg_rec) r = false;   // side-stream events of an earlier backward are not waited for
    m->wg_serial = pt_prof_active();
    const PtcgDims& d = m->dm;
    const DimsX& x = m->dx;
    const int N = m->N, Lt = d.l_tok, NO = d.n_opt, D = d.d, G = d.g;
    const int NL = N * x.l_seq;
    GatherCtx c{m->obs, m->idx, (long)m->off.size, N, d, x, m->off};
    const int* Tr = m->Tr;
    const int* coff = m->compact ? m->c_off : nullptr;
    if (m->compact) {   // the maps of the forward (same rows)
        c.coff = m->c_off; c.rowmap = m->c_map; c.rsam = m->c_rsam; c.rpos = m->c_rpos; c.rows = Tr;
    }
    const bool skip = m->skip_fwd;
    if (skip) {
        c.orow = m->o_row; c.ooff = m->o_off; c.orows = m->o_off + N;
    }
    const int NJo = m->orows;    // option rows of the forward
    const int* Od = m->Odev;
    const int* om = skip ? m->o_row : nullptr;
    const int rows = m->rows;        // trunk launch rows of the forward
    const int* Td = m->Tdev;         // and its device row count (sync-free mode)
    const int tok_rows = m->compact ? rows : N * Lt;

    PT_TRY(pt_fill_zero(m->Gr, m->arena, s));
    PT_TRY(pt_fill_zero(m->dxa, (long)rows * D, s));
    PT_TRY(pt_fill_zero(m->dgd, (long)N * x.bcast_in, s));
    if (d.tables == 1) {
        PT_TRY(pt_fill_zero(m->d_card_vec, (long)d.n_cards * d.d_c, s));
        PT_TRY(pt_fill_zero(m->d_att_tab, (long)d.n_attacks * d.d_a, s));
        PT_TRY(pt_fill_zero(m->d_sk_tab, (long)d.n_skills * d.d_c, s));
    }

    if (d.critic == 1) {
        PT_TRY(critic_bwd(m, c, grad, s));
    } else {
        // blind value head: grad[:, NO] (its weight gradient on the side stream)
        PT_TRY(wg_mark(m, s));
        PT_TRY(pt_head_dot_bwd(grad, 1, NO + 1, NO, m->v2_w, m->v1, m->dv1, N, PT_VAL_H, s));
        PT_TRY(head_dw_side(m, grad, 1, NO + 1, NO, m->v1a, N, PT_VAL_H, m->G(m->v2_w), m->G(m->v2_b), s));
        PT_TRY(wg_mark(m, s));
        PT_TRY(ldx_(m, m->dv1, PT_VAL_H, m->v1_w, m->dvin, x.val_in, N, x.val_in, PT_VAL_H, EPI_STORE, nullptr, 0, s));
        PT_TRY(ldw_side(m, m->dv1, PT_VAL_H, m->val_in, x.val_in, m->G(m->v1_w), m->G(m->v1_b), N, x.val_in, PT_VAL_H, s));
        PT_TRY(pt_val_in_bwd(c, m->dvin, m->dxa, m->dgd, s));
    }

    // option scores: grad[:, :NO] (the weight gradient on the side stream)
    PT_TRY(wg_mark(m, s));
    PT_TRY(pt_head_dot_bwd(grad, NO, NO + 1, 0, m->s2_w, m->s1, m->ds1, NJo, PT_SC_H, s, om, Od));
    PT_TRY(head_dw_side(m, grad, NO, NO + 1, 0, m->s1a, NJo, PT_SC_H, m->G(m->s2_w), m->G(m->s2_b), s, om, Od));
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, m->ds1, PT_SC_H, m->s1_w, m->dsc, x.score_in, NJo, x.score_in, PT_SC_H, EPI_STORE, nullptr, 0, s,
                Od));
    PT_TRY(ldw_side(m, m->ds1, PT_SC_H, m->sc_in, x.score_in, m->G(m->s1_w), m->G(m->s1_b), NJo, x.score_in, PT_SC_H, s,
                Od));
    PT_TRY(pt_sc_in_bwd(c, m->dsc, m->sc_in, m->dq, m->dxa, m->dgd, s));
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, m->dq, D, m->q2_w, m->dq1, D, NJo, D, D, EPI_MUL, m->q1, D, s, Od));
    PT_TRY(ldw_side(m, m->dq, D, m->q1a, D, m->G(m->q2_w), m->G(m->q2_b), NJo, D, D, s, Od));
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, m->dq1, D, m->q1_w, m->dqin, x.q_in, NJo, x.q_in, D, EPI_STORE, nullptr, 0, s, Od));
    PT_TRY(ldw_side(m, m->dq1, D, m->q_in, x.q_in, m->G(m->q1_w), m->G(m->q1_b), NJo, x.q_in, D, s, Od));
    const int oc0 = PT_TYPE_E + 2 * D, oa0 = oc0 + PT_OPT_E;
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, m->dqin + oc0, x.q_in, m->oc_w, m->docard, d.d_c, NJo, d.d_c, PT_OPT_E, EPI_STORE, nullptr, 0, s,
                Od));
    PT_TRY(ldw_side(m, m->dqin + oc0, x.q_in, m->ocard, d.d_c, m->G(m->oc_w), m->G(m->oc_b), NJo, d.d_c, PT_OPT_E, s,
                Od));
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, m->dqin + oa0, x.q_in, m->oa_w, m->doatt, d.d_a, NJo, d.d_a, PT_OPT_E, EPI_STORE, nullptr, 0, s,
                Od));
    PT_TRY(ldw_side(m, m->dqin + oa0, x.q_in, m->oatt, d.d_a, m->G(m->oa_w), m->G(m->oa_b), NJo, d.d_a, PT_OPT_E, s,
                Od));
    // option-type, card and attack table rows of the option rows, then the
    // pointer gradients into the trunk rows (q_in_bwd)
    {
        DetSite S;
        const long nca = (long)d.n_cards * d.d_c, nat = (long)d.n_attacks * d.d_a;
        const int tc = S.add_table(m->dcard, nca, 0, (double)NJo);
        const int ta = S.add_table(m->datt, nat, nca, (double)NJo);
        const int tt = S.add_table(m->G(m->temb), (long)d.n_opt_types * PT_TYPE_E, nca + nat, (double)NJo);
        S.add_source(tc, m->docard, d.d_c, 0, d.d_c, NJo, Od);
        S.add_source(ta, m->doatt, d.d_a, 0, d.d_a, NJo, Od);
        S.add_source(tt, m->dqin, x.q_in, 0, PT_TYPE_E, NJo, Od);
        PT_TRY(pt_det_prepare(m->det, S, s));
        PT_TRY(pt_q_in_bwd(c, m->dqin, m->dxa, pt_det_sink(m->det, S, tt, PT_TYPE_E), s));
        PT_TRY(pt_opt_gather_bwd(c, m->docard, m->doatt, pt_det_sink(m->det, S, tc, d.d_c),
                                 pt_det_sink(m->det, S, ta, d.d_a), s));
        PT_TRY(pt_det_finish(m->det, S, s));
    }

    // final LayerNorm, then the trunk in reverse (d_x in dxb, scratch dxa)
    const bool b16 = m->prec == 1;   // bf16 variant: the LayerNorm also writes dx's bf16 copy (dAh)
    PT_TRY(pt_ln_bwd(m->dxa, D, m->x[d.layers], D, m->lnf_w, m->lnf_mu, m->lnf_rs, nullptr, 0, m->dxb, D,
                     m->G(m->lnf_w), m->G(m->lnf_b), rows, D, m->ws, m->ws_floats, s, Td, b16 ? m->dAh : nullptr));
    for (int i = d.layers - 1; i >= 0; --i)
        PT_TRY(block_bwd(m, m->blk[i], m->ba[i], x.l_seq, m->keep, m->x[i], m->dxb, m->dxa, s, rows, Td, coff,
                         b16 ? &m->bw[i] : nullptr));
    // no join here: nothing after the blocks rewrites what their pending
    // weight gradients read (dxa, dxb, dffn, dqkv, the block activations; the
    // side stream has its own workspace), and the side stream's later work,
    // joined at the end of the backward, runs after them

    // trunk input: readout / token projection / broadcast
    PT_TRY(pt_x0_bwd(c, m->dxb, m->dtokp, m->dbc, s));
    if (m->compact) {
        PT_TRY(pt_gather_rows(m->dxb, D, m->c_off, N, D, m->rd_buf, s));
        PT_TRY(pt_colsum(m->rd_buf, D, N, D, m->G(m->readout), m->ws, m->ws_floats, s));
    } else {
        PT_TRY(pt_colsum(m->dxb, (long)x.l_seq * D, N, D, m->G(m->readout), m->ws, m->ws_floats, s));
    }
    PT_TRY(wg_mark(m, s));
    PT_TRY(ldx_(m, m->dtokp, D, m->tp_w, m->dtokcat, x.tok_in, tok_rows, x.tok_in, D, EPI_STORE, nullptr, 0, s, Td));
    PT_TRY(ldw_side(m, m->dtokp, D, m->tok_cat, x.tok_in, m->G(m->tp_w), m->G(m->tp_b), tok_rows, x.tok_in, D, s, Td));
    // the broadcast product and the decision / global MLPs: their dX products
    // in one launch (the separate products were a chain of small dependent
    // launches); the weight gradients on the side stream once their dY exist
    const MlpChainBwd mb{N, G, PT_DEC_H, x.dec_in, D, m->dbc, m->bc_w, m->g2_w, m->d2_w, m->d1_w, m->g1, m->d1,
                         m->dgd, m->dg1, m->dd1, m->ddec};
    PT_TRY(wg_mark(m, s));
    PT_TRY(pt_mlp_chain_bwd(mb, s));
    PT_TRY(ldw_side(m, m->dbc, D, m->gd, x.bcast_in, m->G(m->bc_w), m->G(m->bc_b), N, x.bcast_in, D, s));
    PT_TRY(wg_mark(m, s));
    // token rows (card, tool cards, zone, owner) and decision slots (select
    // type, context, card, attack) into their tables
    {
        DetSite S;
        const long nca = (long)d.n_cards * d.d_c, nat = (long)d.n_attacks * d.d_a;
        const long nz = (long)d.n_zones * PT_ZONE_E, no = (long)d.n_owners * PT_OWNER_E;
        const long nsl = (long)d.n_select_types * PT_SEL_E;
        const int tc = S.add_table(m->dcard, nca, 0, 3.0 * tok_rows + 4.0 * N);
        const int ta = S.add_table(m->datt, nat, nca, 2.0 * N);
        const int tz = S.add_table(m->G(m->zemb), nz, nca + nat, (double)tok_rows);
        const int to = S.add_table(m->G(m->oemb), no, nca + nat + nz, (double)tok_rows);
        const int tsl = S.add_table(m->G(m->semb), nsl, nca + nat + nz + no, (double)N);
        const int tcx = S.add_table(m->G(m->cemb), (long)d.n_contexts * PT_CTX_E, nca + nat + nz + no + nsl,
                                    (double)N);
        const int* td = m->compact ? Tr : nullptr;
        const int zc = 2 * d.d_c + d.tok_f;   // zone columns of the token concat, then owner
        S.add_source(tc, m->dtokcat, x.tok_in, 0, 2 * d.d_c, tok_rows, td);
        S.add_source(tz, m->dtokcat, x.tok_in, zc, PT_ZONE_E, tok_rows, td);
        S.add_source(to, m->dtokcat, x.tok_in, zc + PT_ZONE_E, PT_OWNER_E, tok_rows, td);
        // decision concat [sel | ctx | 2 card | 2 attack | 2 card | dec_f]
        const int c0 = PT_SEL_E + PT_CTX_E;
        S.add_source(tsl, m->ddec, x.dec_in, 0, PT_SEL_E, N);
        S.add_source(tcx, m->ddec, x.dec_in, PT_SEL_E, PT_CTX_E, N);
        S.add_source(tc, m->ddec, x.dec_in, c0, 2 * d.d_c, N);
        S.add_source(ta, m->ddec, x.dec_in, c0 + 2 * d.d_c, 2 * d.d_a, N);
        S.add_source(tc, m->ddec, x.dec_in, c0 + 2 * d.d_c + 2 * d.d_a, 2 * d.d_c, N);
        PT_TRY(pt_det_prepare(m->det, S, s));
        // decision MLP (d_dvec = dgd[:, G:]) and global MLP (d_g = dgd[:, :G])
        PT_TRY(ldw_side(m, m->dgd + G, x.bcast_in, m->d1a, PT_DEC_H, m->G(m->d2_w), m->G(m->d2_b), N, PT_DEC_H,
                        PT_DEC_H, s));
        PT_TRY(ldw_side(m, m->dd1, PT_DEC_H, m->dec_in, x.dec_in, m->G(m->d1_w), m->G(m->d1_b), N, x.dec_in,
                        PT_DEC_H, s));
        PT_TRY(ldw_side(m, m->dgd, x.bcast_in, m->g1a, G, m->G(m->g2_w), m->G(m->g2_b), N, G, G, s));
        PT_TRY(ldw_side(m, m->dg1, G, m->glob_in, d.global_f, m->G(m->g1_w), m->G(m->g1_b), N, d.global_f, G, s));
        PT_TRY(pt_tok_cat_bwd(c, m->dtokcat, pt_det_sink(m->det, S, tc, d.d_c), pt_det_sink(m->det, S, tz, PT_ZONE_E),
                              pt_det_sink(m->det, S, to, PT_OWNER_E), s));
        PT_TRY(pt_dec_in_bwd(c, m->ddec, pt_det_sink(m->det, S, tc, d.d_c), pt_det_sink(m->det, S, ta, d.d_a),
                             pt_det_sink(m->det, S, tsl, PT_SEL_E), pt_det_sink(m->det, S, tcx, PT_CTX_E), s));
        PT_TRY(pt_det_finish(m->det, S, s));
    }
    if (d.tables == 1) PT_TRY(tables_bwd(m, s));
    return wg_after(m, 5, s);   // join: the heads' and trunk input's weight gradients are done
}
