// Internal interface between the model driver (model.hip) and its kernels.
#pragma once
#include "common.h"

// Section offsets of one obs row (ptcg/rl/buffers.py:212-227).
struct ObsOff {
    int tok_int, tok_float, opt_int, opt_float, opt_mask, global_f, dec_int, dec_float, oracle, size;
};
ObsOff pt_obs_offsets(const PtcgDims& d);

// Width constants of the reference model (ptcg/rl/model.py:114-175).
enum {
    PT_OPT_E = 64, PT_TYPE_E = 16, PT_SC_H = 256, PT_VAL_H = 256, PT_DEC_H = 64,
    PT_ZONE_E = 8, PT_OWNER_E = 4, PT_SEL_E = 8, PT_CTX_E = 32,
};
// Static-table chain (ptcg/rl/model.py:110-127, ptcg_model.cu:38-56): id
// embedding widths, static / text feature widths, pool fan-ins, CardVec MLP.
enum {
    PT_ID_C = 64, PT_ID_A = 48, PT_CARD_STATIC = 58, PT_CARD_TEXT = 128, PT_ATT_STATIC = 15,
    PT_ATT_TEXT = 64, PT_SKILL_TEXT = 64, PT_K_ATT = 4, PT_K_SK = 2, PT_CARD_H = 256,
};
// Oracle block (ptcg/rl/buffers.py:42-45): 24 opp-hand (id, count/4), 24
// split (id, deck/4, prize/4), 8 my-prize (id, count/4) slots; aux-loss
// coefficients and the MY_UNSEEN zone (ptcg_model.cu:83-87).
enum { PT_N_HAND = 24, PT_N_SPLIT = 24, PT_N_PRIZE = 8, PT_ZONE_MY_UNSEEN = 9 };
constexpr float PT_AUX_VF = 1.0f, PT_AUX_HAND = 0.1f, PT_AUX_PRIZE = 0.1f;

struct DimsX {   // derived widths
    int l_seq, dh, tok_in, dec_in, bcast_in, q_in, score_in, val_in;
    int card_in, att_in, sk_in, orc_in, n_orc, l_crit;
};
DimsX pt_dims_x(const PtcgDims& d);

// canonical weight table
struct ParamDef { const char* name; long rows, cols; };
int pt_param_table(const PtcgDims& d, ParamDef* out, int cap);   // returns count or <0

// kernels (layernorm.hip, attention.hip, ppo.hip, adam.hip, gather.hip)
// rows_dev (nullable): device row count <= rows (the launch covers rows)
// ybf: y stored in bf16 (ldy in bf16 elements); dxh (nullable): a bf16 copy of dx
int pt_ln_fwd(const float* x, long ldx, const float* w, const float* b, float* y, long ldy,
              float* mean, float* rstd, int rows, int D, hipStream_t s, const int* rows_dev = nullptr,
              int ybf = 0);
int pt_ln_bwd(const float* dy, long lddy, const float* x, long ldx, const float* w,
              const float* mean, const float* rstd, const float* dres, long ldres, float* dx,
              long lddx, float* dw, float* db, int rows, int D, float* ws, long ws_floats,
              hipStream_t s, const int* rows_dev = nullptr, float* dxh = nullptr);
int pt_attn_supported(int L, int DH);
// coff (nullable): sample n's rows are [coff[n], coff[n+1]) (length <= L);
// else rows n*L .. n*L+L-1.  lse is laid out (N, H, L) either way.
// prec 1: the products (S, P.V and the backward's) on bf16 MFMA with
// operands rounded to bf16, softmax and accumulation in fp32; prec 2: the
// same with qkv, ctx, dctx and dqkv stored in bf16 (pointers reinterpreted).
int pt_attn_fwd(const float* qkv, const float* keep, float* ctx, float* lse, int N, int L, int H,
                int DH, hipStream_t s, const int* coff = nullptr, int prec = 0);
// ws (optional, at least pt_attn_bwd_ws_bytes): global scratch for the
// backward's dS, so that two workgroups fit a CU; without it dS stays in LDS
int pt_attn_bwd(const float* qkv, const float* keep, const float* ctx, const float* lse,
                const float* dctx, float* dqkv, int N, int L, int H, int DH, hipStream_t s,
                const int* coff = nullptr, int prec = 0, void* ws = nullptr, size_t ws_bytes = 0);
size_t pt_attn_bwd_ws_bytes(int N, int L, int H, int DH, int prec);
long pt_ppo_partial_floats(int n);
int pt_ppo_loss(const float* out, int n, int A, const float* mask, long mask_stride,
                const int32_t* idx, const float* actions, const float* old_logp,
                const float* adv, const float* ret, const float* val, const float* prio,
                float clip, float vf_clip, float vf_coef, const float* ent_coef, float* grad,
                float* ratio, float* newvalue, float* stats, float* guard, float* partial,
                hipStream_t s);
int pt_kl_gate(const float* guard, float kl_thr, float vf_thr, float* gate, float* skipped,
               hipStream_t s);
// the sampler with its step read from (and advanced in) device memory
int pt_sample_actions_dev(const float* dec_out, int n, int A, const float* mask, long mask_stride,
                          const int32_t* row_idx, uint64_t seed, uint64_t* step_dev, float* actions,
                          float* logprobs, float* values, hipStream_t s);
// Gumbel-max sampler; noise (n, A) optional (NULL = Philox noise for
// (seed, step or *step_dev, row, option)); step_dev advanced by one when given
int pt_sample_gumbel(const float* dec_out, int n, int A, const float* mask, long mask_stride,
                     const int32_t* row_idx, const float* noise, uint64_t seed, uint64_t step,
                     uint64_t* step_dev, float* actions, float* logprobs, float* values, float* noise_out,
                     hipStream_t s);
struct PtcgMuon;
int pt_muon_set_momentum(PtcgMuon* m, double momentum);
int pt_muon_lr(PtcgMuon* m, float* lr);
long pt_adam_ws_floats();
int pt_adam_step(float* w, float* g, float* m, float* v, long n, const double* lr, double b1, double b2,
                 double eps, float max_norm, const float* gate, int32_t* step, float* norm_out,
                 float* ws, hipStream_t s);
int pt_adam_step(float* w, float* g, float* m, float* v, long n, const float* lr, double b1, double b2,
                 double eps, float max_norm, const float* gate, int32_t* step, float* norm_out,
                 float* ws, hipStream_t s);

// ---- bf16 copies (bf16copy.hip)
// One weight matrix W (rows = out, cols = in): dst = bf16 W, dstT = bf16 W^T
// (cols x rows).  tile0 is set by pt_bf16_weights.
struct BfWeight { const float* src; __bf16* dst; __bf16* dstT; int rows, cols, tile0; };
constexpr int BF_MAX_W = 24;
struct BfWeightSet { int n = 0; BfWeight m[BF_MAX_W]; };
int pt_bf16_weights(BfWeightSet& ws, hipStream_t s);
// n floats of src to bf16 at dst (reinterpreted as __bf16)
int pt_to_bf16(const float* src, float* dst, long n, hipStream_t s);

// ---- order-independent table scatters (detsum.hip)
// A site: the tables one point of the backward scatters into and the
// gradient slices it scatters from (sources; source i feeds table stab[i]).
constexpr int DET_MAX_TAB = 8, DET_MAX_SRC = 8, DET_PART = 256;
struct DetSite {
    int ntab = 0;
    float* tab[DET_MAX_TAB] = {};       // float tables (the grads), += at finish
    long tab_n[DET_MAX_TAB] = {};       // floats per table
    long acc_off[DET_MAX_TAB] = {};     // their accumulators in DetCtx::acc
    double count[DET_MAX_TAB] = {};     // contributions one element can receive (bound)
    int nsrc = 0;
    const float* sp[DET_MAX_SRC] = {};  // source rows: sp + r * sld + scol, swidth floats,
    long sld[DET_MAX_SRC] = {};         // r < min(srows, *srows_dev)
    int scol[DET_MAX_SRC] = {}, swidth[DET_MAX_SRC] = {}, stab[DET_MAX_SRC] = {};
    int svec[DET_MAX_SRC] = {};         // set by pt_det_prepare: 128-bit loads allowed
    long srows[DET_MAX_SRC] = {};
    const int* srows_dev[DET_MAX_SRC] = {};
    int add_table(float* t, long n, long off, double cnt) {
        tab[ntab] = t; tab_n[ntab] = n; acc_off[ntab] = off; count[ntab] = cnt < 1.0 ? 1.0 : cnt;
        return ntab++;
    }
    void add_source(int t, const float* p, long ld, int col, int width, long rows, const int* rows_dev = nullptr) {
        sp[nsrc] = p; sld[nsrc] = ld; scol[nsrc] = col; swidth[nsrc] = width; srows[nsrc] = rows;
        srows_dev[nsrc] = rows_dev; stab[nsrc] = t; ++nsrc;
    }
};
// the model's accumulator memory (zero between sites), per-block maxima, scales
struct DetCtx { unsigned long long* acc; long acc_len; float* part; double* scale; };
// where a scatter kernel adds table t's contributions: row-major, ld floats per id
struct DetSink { unsigned long long* acc; const double* scale; long ld; };
int pt_det_prepare(const DetCtx& d, const DetSite& S, hipStream_t s);   // absmax + scales
int pt_det_finish(const DetCtx& d, const DetSite& S, hipStream_t s);    // tables += acc, acc = 0
DetSink pt_det_sink(const DetCtx& d, const DetSite& S, int t, long ld);
// fixed-point add of an fp32 partial sum into element e of a sink (scale read
// by the caller once per thread; scale < 0 marks a non-finite table)
__device__ __forceinline__ void pt_det_add(const DetSink& k, double scale, long e, float a) {
    if (a != 0.f && scale > 0.0 && isfinite(a))
        atomicAdd(k.acc + e, (unsigned long long)(long long)rint((double)a * scale));
}

// ---- gathers / scatters of the token, decision and option paths (gather.hip)
struct GatherCtx {
    const float* obs; const int32_t* idx; long stride; int N;
    PtcgDims dm; DimsX dx; ObsOff off;
    // compact trunk layout (null = full length, row n*l_seq + pos): sample n
    // owns rows [coff[n], coff[n+1]) = READOUT then its active positions
    // (valid tokens and pointer targets) in order; rowmap[n*l_seq + pos] is
    // the row of an active position (-1 otherwise); rsam / rpos invert it;
    // *rows = coff[N].
    const int* coff; const int* rowmap; const int* rsam; const int* rpos; const int* rows;
    // compact option rows (null = all n_opt options, row n*n_opt + j): sample
    // n's legal options (every option when it has none legal) are rows
    // [ooff[n], ooff[n+1]) in slot order; orow[i] = n*n_opt + j of row i;
    // *orows = ooff[N]
    const int* orow; const int* ooff; const int* orows;
};
// option (n * n_opt + j) of option row i
__device__ __forceinline__ long pt_onj(const GatherCtx& c, long i) { return c.orow ? (long)c.orow[i] : i; }
// option rows of the launch: the device count bounds the compact layout
__device__ __forceinline__ long pt_orows(const GatherCtx& c) {
    return c.orow ? (long)*c.orows : (long)c.N * c.dm.n_opt;
}
// trunk row of (sample n, position pos); pos must be active in the compact layout
__device__ __forceinline__ long pt_hrow(const GatherCtx& c, int n, int pos) {
    return c.rowmap ? (long)c.rowmap[(long)n * c.dx.l_seq + pos] : (long)n * c.dx.l_seq + pos;
}
int pt_tok_cat_fwd(const GatherCtx& c, const float* card, const float* zemb, const float* oemb,
                   float* tok_cat, hipStream_t s,
                   long rows_done = 0);
int pt_tok_cat_bwd(const GatherCtx& c, const float* d_cat, const DetSink& d_card, const DetSink& d_zemb,
                   const DetSink& d_oemb, hipStream_t s);
int pt_glob_in(const GatherCtx& c, float* glob_in, hipStream_t s);
// The global MLP, decision MLP and broadcast product of B samples in one
// launch (mlpchain.hip): inputs glob_in (N x gf), dec_in (N x din); weights
// (out, in) row-major; outputs g1 = gelu'(z1), g1a = gelu(z1) (N x G), d1 / d1a
// (N x H), gd = [g | d] (N x (G + H)), bc (N x D)
struct MlpChain {
    int N, gf, G, din, H, D;
    const float *glob_in, *dec_in;
    const float *g1w, *g1b, *g2w, *g2b, *d1w, *d1b, *d2w, *d2b, *bcw, *bcb;
    float *g1, *g1a, *d1, *d1a, *gd, *bc;
};
bool pt_mlp_chain_fits(const MlpChain& a);
int pt_mlp_chain_fwd(const MlpChain& a, hipStream_t s);
// the chain's dX products in one launch: dgd (N x (G + H)) += dbc (N x D) Wb,
// dd1 = (dgd[:, G:] W4) * d1, ddec = dd1 W3 (N x din), dg1 = (dgd[:, :G] W2) * g1
struct MlpChainBwd {
    int N, G, H, din, D;
    const float *dbc, *bcw, *g2w, *d2w, *d1w, *g1, *d1;
    float *dgd, *dg1, *dd1, *ddec;
};
int pt_mlp_chain_bwd(const MlpChainBwd& a, hipStream_t s);
int pt_dec_in_fwd(const GatherCtx& c, const float* card, const float* att, const float* semb,
                  const float* cemb, float* dec_in, hipStream_t s);
int pt_dec_in_bwd(const GatherCtx& c, const float* d_in, const DetSink& d_card, const DetSink& d_att,
                  const DetSink& d_semb, const DetSink& d_cemb, hipStream_t s);
// lny (nullable, d = 256): the first block's LayerNorm 1 of x0 in the same
// launch (lnybf: bf16 output), with its mean / rstd
int pt_x0_fwd(const GatherCtx& c, const float* tokp, const float* bc, const float* readout,
              float* x0, float* keep, hipStream_t s, const float* lnw = nullptr, const float* lnb = nullptr,
              float* lny = nullptr, float* lnmu = nullptr, float* lnrs = nullptr, int lnybf = 0);
int pt_x0_bwd(const GatherCtx& c, const float* d_x0, float* d_tokp, float* d_bc, hipStream_t s);
int pt_opt_gather_fwd(const GatherCtx& c, const float* card, const float* att, float* ocard,
                      float* oatt, hipStream_t s);
int pt_opt_gather_bwd(const GatherCtx& c, const float* d_ocard, const float* d_oatt,
                      const DetSink& d_card, const DetSink& d_att, hipStream_t s);
int pt_q_in_fwd(const GatherCtx& c, const float* h, const float* temb, float* q_in, hipStream_t s);
int pt_q_in_bwd(const GatherCtx& c, const float* d_qin, float* d_h, const DetSink& d_temb, hipStream_t s);
int pt_sc_in_fwd(const GatherCtx& c, const float* h, const float* gd, float* sc_in, hipStream_t s);
int pt_sc_in_bwd(const GatherCtx& c, const float* d_sc, const float* sc_in, float* d_q,
                 float* d_h, float* d_gd, hipStream_t s);
// [seq[:, 0] | g] over sequences of ls rows (ls = 0: the trunk's l_seq)
int pt_val_in_fwd(const GatherCtx& c, const float* h, const float* gd, float* val_in, hipStream_t s, int ls = 0);
int pt_val_in_bwd(const GatherCtx& c, const float* d_val_in, float* d_h, float* d_gd, hipStream_t s, int ls = 0);
// y[r] = X[r,:] . w + b, written to out[q / per * ldo + col0 + q % per], q = rmap ? rmap[r] : r;
// rows_dev (nullable): device row count <= rows
int pt_head_dot(const float* X, int rows, int K, const float* w, const float* b, float* out,
                int per, long ldo, int col0, hipStream_t s, const int* rmap = nullptr,
                const int* rows_dev = nullptr);
// dX[r,:] = dy[r] * w[:] * gd[r,:] (gd = the GELU derivative kept by the forward),
// dy[r] = grad[q / per * ldg + col0 + q % per]
int pt_head_dot_bwd(const float* grad, int per, long ldg, int col0, const float* w,
                    const float* gd, float* dX, int rows, int K, hipStream_t s, const int* rmap = nullptr,
                    const int* rows_dev = nullptr);
// dw[k] = sum_r dy[r] X[r,k]; db = sum_r dy[r]   (fixed order)
int pt_head_dot_dw(const float* grad, int per, long ldg, int col0, const float* X, int rows, int K,
                   float* dw, float* db, float* ws, long ws_floats, hipStream_t s, const int* rmap = nullptr,
                   const int* rows_dev = nullptr);
int pt_fill_zero(float* p, long n, hipStream_t s);

// ---- reference model variant: static tables, oracle critic, aux losses (frozen.hip)
int pt_copy_cols(float* dst, long ldd, const float* src, long lds, int rows, int cols, hipStream_t s);
int pt_pool_fwd(const float* tab, int E, const int* ids, int K, int NC, float* out, long ldo, int col_mean,
                int col_max, int* amax, hipStream_t s);
int pt_pool_bwd(const float* dsrc, long ld, int col_mean, int col_max, const int* amax, const int* ids, int K,
                int NC, int E, const DetSink& d_tab, hipStream_t s);
// dx = dy * gd elementwise (gd = the GELU derivative kept by the forward)
int pt_mul(const float* dy, const float* gd, float* dx, long n, hipStream_t s);
int pt_otok_in(const GatherCtx& c, const float* cv, const float* keep, float* out, float* ckeep, hipStream_t s);
int pt_otok_bwd(const GatherCtx& c, const float* d_in, const DetSink& d_card, hipStream_t s);
int pt_xc_fwd(const float* cread, const float* h, const float* otok, float* xc, int N, int Ls, int NO, int D,
              hipStream_t s);
int pt_xc_bwd(const float* d_xc, float* d_h, float* d_otok, int N, int Ls, int NO, int D, hipStream_t s);
int pt_aux_grads(const GatherCtx& c, const float* hand_lin, const float* prize_all, const float* blind_v,
                 const float* ret, int* cnt, float* d_hand, float* d_prize, float* d_blind, hipStream_t s);
int pt_rank1_add(const float* dy, const float* w, float* dX, int rows, int K, hipStream_t s);

// ---- compact trunk layout (compact.hip)
// Active positions of each sample (READOUT, valid tokens, pointer targets),
// row offsets, row maps; act is scratch of N * l_seq ints.
int pt_compact_map(const GatherCtx& c, int* act, int* cnt, int* coff, int* rowmap, int* rsam, int* rpos,
                   hipStream_t s);
// Option rows of each sample: its legal options (opt_mask != 0), or all of
// them when none is legal; per-sample counts, offsets, row -> option map.
int pt_opt_map(const GatherCtx& c, int* cnt, int* ooff, int* orow, hipStream_t s);
// dst[n] = src[coff[n]]  (rows of width D)
int pt_gather_rows(const float* src, long ld, const int* coff, int N, int D, float* dst, hipStream_t s);
