// Gathers and scatters around the GEMMs: token concat, decision concat,
// trunk input assembly, option-scorer inputs, and their backward scatters.
//
// Reference counterparts (native/model/ptcg_model.cu, ptcg_model2.cu):
//   k_tok_cat :289 / k_tok_cat_bwd :36      -> tok_cat_*
//   k_dec_in :324 / k_dec_in_bwd :66        -> dec_in_*
//   k_x0 :348 / k_x0_bwd :202               -> x0_*
//   k_opt_gather :371 / k_opt_gather_bwd :135
//   k_q_in :390 / k_q_in_bwd :85
//   k_sc_in :423 / k_sc_in_bwd :115
//   k_val_in :503 / k_val_in_bwd :191
// Ids come from fp32 obs columns: (int) truncation toward zero, then clamp
// to the vocabulary (ptcg_model.cu:299-318).  Forward gathers move 16 B per
// lane.  Per-sample reductions (the bcast row sum, the pointer scatter into
// the trunk output, the option sums into r/g/dvec) run one workgroup per
// sample, each element owned by one thread; the scatters into shared
// embedding tables (card/attack/zone/owner/type/select/context rows shared
// across samples), where the reference uses fp32 atomics, sum rows of equal
// id in a per-thread id cache (IdCache) and add the partial sums in 64-bit
// fixed point (detsum.hip), so the tables' gradients do not depend on the
// order the adds land in.
#include "model.h"

#include <algorithm>

namespace {

constexpr int TB = 256;
constexpr int PT_MAX_OPT = 256;   // options per sample the q_in backward stages in LDS

// TOK_LPR lanes per row (256 / TOK_LPR rows per workgroup): a row's metadata
// (sample, position, obs row, token ids) is loaded once per lane group — the
// same address in its lanes — and the group walks the row's 16-byte chunks;
// 64 / TOK_LPR rows per wave keep that many dependent lookup chains in flight.
constexpr int TOK_LPR = 8;
__global__ void tok_cat_fwd_kernel(GatherCtx c, const float* __restrict__ card,
        const float* __restrict__ zemb, const float* __restrict__ oemb, float* __restrict__ out) {
    const int Lt = c.dm.l_tok, dc = c.dm.d_c, tin = c.dx.tok_in;
    const int chunks = tin / 4;
    const int lane = threadIdx.x % TOK_LPR;
    const long r = (long)blockIdx.x * (TB / TOK_LPR) + threadIdx.x / TOK_LPR;
    // rows: (n, token t) full length, or the compact trunk rows (READOUT rows get zeros)
    const long nrows = c.rowmap ? (long)*c.rows : (long)c.N * Lt;
    if (r >= nrows) return;
    int n, t;
    if (c.rowmap) {
        n = c.rsam[r];
        t = c.rpos[r] - 1;
        if (t < 0) {
            for (int ch = lane; ch < chunks; ch += TOK_LPR)
                *reinterpret_cast<float4*>(out + r * tin + ch * 4) = make_float4(0.f, 0.f, 0.f, 0.f);
            return;
        }
    } else {
        n = (int)(r / Lt);
        t = (int)(r % Lt);
    }
    const float* row = obs_row(c.obs, c.idx, c.stride, n);
    const float* ti = row + c.off.tok_int + (long)t * c.dm.tok_int;
    const int NC = c.dm.n_cards;
    const int cid = pt_id_clamp(ti[0], NC - 1);
    const int t0 = (int)ti[3], t1 = (int)ti[4];
    const int z = pt_id_clamp(ti[1], c.dm.n_zones - 1);
    const int o = pt_id_clamp(ti[2], c.dm.n_owners - 1);
    for (int ch = lane; ch < chunks; ch += TOK_LPR) {
        const int col = ch * 4;
        float4 v;
        if (col < dc) {
            v = *reinterpret_cast<const float4*>(card + (long)cid * dc + col);
        } else if (col < 2 * dc) {
            const int e = col - dc;
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
            if (t0 > 0) a = *reinterpret_cast<const float4*>(card + (long)(t0 >= NC ? NC - 1 : t0) * dc + e);
            if (t1 > 0) b = *reinterpret_cast<const float4*>(card + (long)(t1 >= NC ? NC - 1 : t1) * dc + e);
            v = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
        } else if (col < 2 * dc + c.dm.tok_f) {
            v = *reinterpret_cast<const float4*>(row + c.off.tok_float + (long)t * c.dm.tok_f + (col - 2 * dc));
        } else if (col < 2 * dc + c.dm.tok_f + PT_ZONE_E) {
            v = *reinterpret_cast<const float4*>(zemb + z * PT_ZONE_E + (col - 2 * dc - c.dm.tok_f));
        } else {
            v = *reinterpret_cast<const float4*>(oemb + o * PT_OWNER_E + (col - 2 * dc - c.dm.tok_f - PT_ZONE_E));
        }
        *reinterpret_cast<float4*>(out + r * tin + col) = v;
    }
}

// Scatter-add of one table column with a per-thread cache of four (id, sum)
// pairs.  A thread walks its column down a run of rows in order; rows that
// share an id (padding ids, the few zones / owners / option types, frequent
// cards) add in registers, and the table sees one fixed-point add (pt_det_add)
// per eviction instead of one per row — the reference's per-element atomics
// serialise on such hot rows.  Zero gradients (masked options, padding) are
// skipped.
struct IdCache {
    int id0 = -1, id1 = -1, id2 = -1, id3 = -1;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int next = 0;
    DetSink k;
    double sc;
    int col;
    __device__ IdCache(const DetSink& sink, int col_) : k(sink), sc(*sink.scale), col(col_) {}
    __device__ __forceinline__ void put(int id, float a) {
        if (id >= 0) pt_det_add(k, sc, (long)id * k.ld + col, a);
    }
    __device__ __forceinline__ void add(int id, float g) {
        if (g == 0.f) return;
        if (id == id0) { a0 += g; return; }
        if (id == id1) { a1 += g; return; }
        if (id == id2) { a2 += g; return; }
        if (id == id3) { a3 += g; return; }
        if (next == 0) { put(id0, a0); id0 = id; a0 = g; }
        else if (next == 1) { put(id1, a1); id1 = id; a1 = g; }
        else if (next == 2) { put(id2, a2); id2 = id; a2 = g; }
        else { put(id3, a3); id3 = id; a3 = g; }
        next = (next + 1) & 3;
    }
    __device__ __forceinline__ void flush() {
        put(id0, a0);
        put(id1, a1);
        put(id2, a2);
        put(id3, a3);
    }
};

// rows per workgroup of the column-owner scatters
constexpr int SCATTER_ROWS = 32;

// token concat backward: thread = one gradient-bearing column (card | tool
// card | zone | owner; the numeric features are inputs), workgroup = a run
// of SCATTER_ROWS token rows
__global__ void tok_cat_bwd_kernel(GatherCtx c, const float* __restrict__ d_cat, DetSink d_card, DetSink d_zemb,
                                   DetSink d_oemb) {
    const int Lt = c.dm.l_tok, dc = c.dm.d_c, tin = c.dx.tok_in;
    const int zc = 2 * dc + c.dm.tok_f;   // first zone column of the concat
    const int q = threadIdx.x;
    if (q >= 2 * dc + PT_ZONE_E + PT_OWNER_E) return;
    const int col = q < 2 * dc ? q : zc + (q - 2 * dc);
    const long nrows = c.rowmap ? (long)*c.rows : (long)c.N * Lt;
    const long r0 = (long)blockIdx.x * SCATTER_ROWS, r1 = min(nrows, r0 + SCATTER_ROWS);
    const int NC = c.dm.n_cards;
    const int tc = q < dc ? q : (q < 2 * dc ? q - dc : (q < 2 * dc + PT_ZONE_E ? q - 2 * dc : q - 2 * dc - PT_ZONE_E));
    const DetSink& sk = q < 2 * dc ? d_card : (q < 2 * dc + PT_ZONE_E ? d_zemb : d_oemb);
    IdCache k0(sk, tc), k1(sk, tc);   // k1: the second tool card
    for (long r = r0; r < r1; ++r) {
        const float g = d_cat[r * tin + col];
        if (g == 0.f) continue;
        int n, t;
        if (c.rowmap) {
            n = c.rsam[r];
            t = c.rpos[r] - 1;
            if (t < 0) continue;
        } else {
            n = (int)(r / Lt);
            t = (int)(r % Lt);
        }
        const float* ti = obs_row(c.obs, c.idx, c.stride, n) + c.off.tok_int + (long)t * c.dm.tok_int;
        if (q < dc) {
            k0.add(pt_id_clamp(ti[0], NC - 1), g);
        } else if (q < 2 * dc) {
            const int t0 = (int)ti[3], t1 = (int)ti[4];
            if (t0 > 0) k0.add(t0 >= NC ? NC - 1 : t0, g);
            if (t1 > 0) k1.add(t1 >= NC ? NC - 1 : t1, g);
        } else if (q < 2 * dc + PT_ZONE_E) {
            k0.add(pt_id_clamp(ti[1], c.dm.n_zones - 1), g);
        } else {
            k0.add(pt_id_clamp(ti[2], c.dm.n_owners - 1), g);
        }
    }
    k0.flush();
    k1.flush();
}

// rows (or samples, options) whose loads are issued together before their
// ordered adds, in the scatters bound by a chain of dependent loads per row
constexpr int PF = 16;

__global__ void glob_in_kernel(GatherCtx c, float* __restrict__ out) {
    const int G = c.dm.global_f;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)c.N * G) return;
    const int n = (int)(i / G), k = (int)(i % G);
    out[i] = obs_row(c.obs, c.idx, c.stride, n)[c.off.global_f + k];
}

// dec concat: [sel8 | ctx32 | cv(eff) | cv(ctx) | av(my) | av(opp) | cv(msup) | cv(osup) | dec_f]
struct DecSeg { int kind; int slot; int width; };
__device__ __forceinline__ void dec_locate(const GatherCtx& c, int col, int& kind, int& di, int& e) {
    const int dc = c.dm.d_c, da = c.dm.d_a;
    const int b0 = PT_SEL_E, b1 = b0 + PT_CTX_E, b2 = b1 + dc, b3 = b2 + dc, b4 = b3 + da,
              b5 = b4 + da, b6 = b5 + dc, b7 = b6 + dc;
    if (col < b0) { kind = 0; di = 0; e = col; }
    else if (col < b1) { kind = 1; di = 1; e = col - b0; }
    else if (col < b2) { kind = 2; di = 2; e = col - b1; }
    else if (col < b3) { kind = 2; di = 3; e = col - b2; }
    else if (col < b4) { kind = 3; di = 4; e = col - b3; }
    else if (col < b5) { kind = 3; di = 5; e = col - b4; }
    else if (col < b6) { kind = 2; di = 6; e = col - b5; }
    else if (col < b7) { kind = 2; di = 7; e = col - b6; }
    else { kind = 4; di = 0; e = col - b7; }
}

__global__ void dec_in_fwd_kernel(GatherCtx c, const float* __restrict__ card,
        const float* __restrict__ att, const float* __restrict__ semb,
        const float* __restrict__ cemb, float* __restrict__ out) {
    const int W = c.dx.dec_in;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)c.N * W) return;
    const int n = (int)(i / W), col = (int)(i % W);
    const float* row = obs_row(c.obs, c.idx, c.stride, n);
    const float* di_ = row + c.off.dec_int;
    int kind, di, e;
    dec_locate(c, col, kind, di, e);
    float v;
    if (kind == 0) v = semb[pt_id_clamp(di_[0], c.dm.n_select_types - 1) * PT_SEL_E + e];
    else if (kind == 1) v = cemb[pt_id_clamp(di_[1], c.dm.n_contexts - 1) * PT_CTX_E + e];
    else if (kind == 2) v = card[(long)pt_id_clamp(di_[di], c.dm.n_cards - 1) * c.dm.d_c + e];
    else if (kind == 3) v = att[(long)pt_id_clamp(di_[di], c.dm.n_attacks - 1) * c.dm.d_a + e];
    else v = row[c.off.dec_float + e];
    out[i] = v;
}

// decision concat backward: thread = column, workgroup = (column block, a
// run of SCATTER_ROWS samples)
__global__ void dec_in_bwd_kernel(GatherCtx c, const float* __restrict__ d_in, DetSink d_card, DetSink d_att,
                                  DetSink d_semb, DetSink d_cemb) {
    const int W = c.dx.dec_in;
    const int col = blockIdx.x * TB + threadIdx.x;
    if (col >= W) return;
    int kind, di, e;
    dec_locate(c, col, kind, di, e);
    if (kind == 4) return;   // numeric features: no gradient
    const DetSink& sk = kind == 0 ? d_semb : (kind == 1 ? d_cemb : (kind == 2 ? d_card : d_att));
    const int hi = kind == 0 ? c.dm.n_select_types - 1
                 : (kind == 1 ? c.dm.n_contexts - 1 : (kind == 2 ? c.dm.n_cards - 1 : c.dm.n_attacks - 1));
    const int n0 = blockIdx.y * SCATTER_ROWS, n1 = min(c.N, n0 + SCATTER_ROWS);
    IdCache k(sk, e);
    for (int n = n0; n < n1; ++n) {
        const float g = d_in[(long)n * W + col];
        if (g == 0.f) continue;
        const float* di_ = obs_row(c.obs, c.idx, c.stride, n) + c.off.dec_int;
        k.add(pt_id_clamp(di_[di], hi), g);
    }
    k.flush();
}

// x0[n,0] = readout; x0[n,l] = tokp[n,l-1] + bc[n]; keep[n,l] = l==0 || zone_float > 0
// lny (nullable, d = 256): also the first block's LayerNorm 1 of the row, in
// ln_fwd_kernel's arithmetic (a wave holds one row, one float4 per lane), into
// lny (bf16 when lnybf) with its mean / rstd
__global__ void x0_fwd_kernel(GatherCtx c, const float* __restrict__ tokp,
        const float* __restrict__ bc, const float* __restrict__ readout, float* __restrict__ x0,
        float* __restrict__ keep, const float* __restrict__ lnw, const float* __restrict__ lnb,
        float* __restrict__ lny, float* __restrict__ lnmu, float* __restrict__ lnrs, int lnybf) {
    const int Ls = c.dx.l_seq, D = c.dm.d, ch4 = D / 4;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    const long nrows = c.rowmap ? (long)*c.rows : (long)c.N * Ls;
    if (i >= nrows * ch4) return;
    const int col = (int)(i % ch4) * 4;
    const long nl = i / ch4;
    // full length: row (n, l), token projection row (n, l-1); compact: both at row nl
    const int n = c.rowmap ? c.rsam[nl] : (int)(nl / Ls), l = c.rowmap ? c.rpos[nl] : (int)(nl % Ls);
    float4 v;
    if (l == 0) {
        v = *reinterpret_cast<const float4*>(readout + col);
    } else {
        const long tr = c.rowmap ? nl : (long)n * c.dm.l_tok + (l - 1);
        const float4 a = *reinterpret_cast<const float4*>(tokp + tr * D + col);
        const float4 b = *reinterpret_cast<const float4*>(bc + (long)n * D + col);
        v = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    }
    *reinterpret_cast<float4*>(x0 + nl * D + col) = v;
    if (lny) {
        const float mu = wave_sum((v.x + v.y) + (v.z + v.w)) / (float)D;
        const float a = v.x - mu, b = v.y - mu, cc = v.z - mu, dd = v.w - mu;
        const float var = wave_sum((a * a + b * b) + (cc * cc + dd * dd)) / (float)D;
        const float rs = 1.0f / sqrtf(var + 1e-5f);
        if (col == 0) {
            lnmu[nl] = mu;
            lnrs[nl] = rs;
        }
        const float4 ww = *reinterpret_cast<const float4*>(lnw + col);
        const float4 wb = *reinterpret_cast<const float4*>(lnb + col);
        float4 o;
        o.x = (v.x - mu) * rs * ww.x + wb.x;
        o.y = (v.y - mu) * rs * ww.y + wb.y;
        o.z = (v.z - mu) * rs * ww.z + wb.z;
        o.w = (v.w - mu) * rs * ww.w + wb.w;
        if (lnybf) {
            typedef __bf16 x0bf16x4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<x0bf16x4*>(reinterpret_cast<__bf16*>(lny) + nl * D + col) =
                x0bf16x4{(__bf16)o.x, (__bf16)o.y, (__bf16)o.z, (__bf16)o.w};
        } else {
            *reinterpret_cast<float4*>(lny + nl * D + col) = o;
        }
    }
    if (col == 0) {
        float kp = 1.f;
        if (l > 0) {
            const float z = obs_row(c.obs, c.idx, c.stride, n)[c.off.tok_int + (long)(l - 1) * c.dm.tok_int + 1];
            kp = z > 0.f ? 1.f : 0.f;
        }
        keep[nl] = kp;
    }
}

// one workgroup per sample: d_tokp[n,t] = d_x0[n,t+1]; d_bc[n] = sum_t d_x0[n,t+1]
__global__ void x0_bwd_kernel(GatherCtx c, const float* __restrict__ d_x0, float* __restrict__ d_tokp,
                              float* __restrict__ d_bc) {
    const int n = blockIdx.x, Ls = c.dx.l_seq, Lt = c.dm.l_tok, D = c.dm.d;
    if (c.rowmap) {   // compact: the sample's rows after its READOUT row (token rows share the index)
        const long r0 = c.coff[n], r1 = c.coff[n + 1];
        for (int col = threadIdx.x; col < D; col += TB) {
            float acc = 0.f;
            d_tokp[r0 * D + col] = 0.f;
            for (long rb = r0 + 1; rb < r1; rb += PF) {   // PF rows' loads together, sums in row order
                float v[PF];
#pragma unroll
                for (int u = 0; u < PF; ++u) v[u] = rb + u < r1 ? d_x0[(rb + u) * D + col] : 0.f;
#pragma unroll
                for (int u = 0; u < PF; ++u) {
                    if (rb + u >= r1) break;
                    d_tokp[(rb + u) * D + col] = v[u];
                    acc += v[u];
                }
            }
            d_bc[(long)n * D + col] = acc;
        }
        return;
    }
    for (int col = threadIdx.x; col < D; col += TB) {
        float acc = 0.f;
        for (int t = 0; t < Lt; ++t) {
            const float v = d_x0[((long)n * Ls + t + 1) * D + col];
            d_tokp[((long)n * Lt + t) * D + col] = v;
            acc += v;
        }
        d_bc[(long)n * D + col] = acc;
    }
}

__global__ void opt_gather_fwd_kernel(GatherCtx c, const float* __restrict__ card,
        const float* __restrict__ att, float* __restrict__ ocard, float* __restrict__ oatt) {
    const int NO = c.dm.n_opt, dc = c.dm.d_c, da = c.dm.d_a;
    const int W = dc > da ? dc : da;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= pt_orows(c) * W) return;
    const int e = (int)(i % W);
    const long row = i / W, nj = pt_onj(c, row);   // option row, option
    const int n = (int)(nj / NO), j = (int)(nj % NO);
    const float* oi = obs_row(c.obs, c.idx, c.stride, n) + c.off.opt_int + (long)j * c.dm.opt_int;
    if (e < dc) ocard[row * dc + e] = card[(long)pt_id_clamp(oi[3], c.dm.n_cards - 1) * dc + e];
    if (e < da) oatt[row * da + e] = att[(long)pt_id_clamp(oi[4], c.dm.n_attacks - 1) * da + e];
}

// option card / attack backward: thread = column (d_c card columns, then
// d_a attack columns), workgroup = a run of SCATTER_ROWS options
__global__ void opt_gather_bwd_kernel(GatherCtx c, const float* __restrict__ d_ocard,
        const float* __restrict__ d_oatt, DetSink d_card, DetSink d_att) {
    const int NO = c.dm.n_opt, dc = c.dm.d_c, da = c.dm.d_a;
    const int q = threadIdx.x;
    if (q >= dc + da) return;
    const bool is_card = q < dc;
    const int e = is_card ? q : q - dc;
    const int w = is_card ? dc : da;
    const float* src = is_card ? d_ocard : d_oatt;
    const int hi = is_card ? c.dm.n_cards - 1 : c.dm.n_attacks - 1;
    const int slot = is_card ? 3 : 4;
    const long r0 = (long)blockIdx.x * SCATTER_ROWS, r1 = min(pt_orows(c), r0 + SCATTER_ROWS);
    IdCache k(is_card ? d_card : d_att, e);
    for (long row = r0; row < r1; ++row) {
        const float g = src[row * w + e];
        if (g == 0.f) continue;
        const long nj = pt_onj(c, row);
        const int n = (int)(nj / NO), j = (int)(nj % NO);
        const float* oi = obs_row(c.obs, c.idx, c.stride, n) + c.off.opt_int + (long)j * c.dm.opt_int;
        k.add(pt_id_clamp(oi[slot], hi), g);
    }
    k.flush();
}

// q_in = [temb16 | h(p1) | h(p2) | (opt_card, opt_attack GEMM outputs) | opt_f]
__global__ void q_in_fwd_kernel(GatherCtx c, const float* __restrict__ h,
        const float* __restrict__ temb, float* __restrict__ q_in) {
    const int NO = c.dm.n_opt, D = c.dm.d, W = c.dx.q_in, ch = W / 4;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= pt_orows(c) * ch) return;
    const int col = (int)(i % ch) * 4;
    const long orow = i / ch, nj = pt_onj(c, orow);   // option row, option
    const int n = (int)(nj / NO), j = (int)(nj % NO);
    const int oc0 = PT_TYPE_E + 2 * D, of0 = oc0 + 2 * PT_OPT_E;
    if (col >= oc0 && col < of0) return;      // written by the opt_card / opt_attack GEMMs
    const float* row = obs_row(c.obs, c.idx, c.stride, n);
    const float* oi = row + c.off.opt_int + (long)j * c.dm.opt_int;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (col < PT_TYPE_E) {
        v = *reinterpret_cast<const float4*>(temb + pt_id_clamp(oi[0], c.dm.n_opt_types - 1) * PT_TYPE_E + col);
    } else if (col < oc0) {
        const int which = col < PT_TYPE_E + D ? 1 : 2;
        const int e = col - PT_TYPE_E - (which - 1) * D;
        const int p = (int)oi[which];      // 0 = null; else trunk position p (token p-1)
        if (p > 0 && p <= c.dm.l_tok)
            v = *reinterpret_cast<const float4*>(h + pt_hrow(c, n, p) * D + e);
    } else {
        v = *reinterpret_cast<const float4*>(row + c.off.opt_float + (long)j * c.dm.opt_f + (col - of0));
    }
    *reinterpret_cast<float4*>(q_in + orow * W + col) = v;
}

// one workgroup per sample: d_h[n,p] += d_qin pointer slices.  A thread
// owns its columns, so no two threads add to one element; the adds are
// no-return atomics so successive options do not wait on each other's
// read-modify-write.  Option types (few, hot) go through an id cache.
// One workgroup per sample.  The sample's option rows' lookups (option slot
// -> option ids -> trunk rows of the two pointer targets) are resolved once
// into LDS; each thread then walks the options in order for its column, so
// a column's atomics keep their order (deterministic sums) while the
// gradient loads of successive options no longer wait on a lookup chain.
__global__ void q_in_bwd_kernel(GatherCtx c, const float* __restrict__ d_qin, float* __restrict__ d_h,
                                DetSink d_temb) {
    __shared__ long s_h1[PT_MAX_OPT], s_h2[PT_MAX_OPT];
    __shared__ int s_ty[PT_MAX_OPT];
    const int n = blockIdx.x, NO = c.dm.n_opt, D = c.dm.d, W = c.dx.q_in;
    const float* row = obs_row(c.obs, c.idx, c.stride, n);
    // the sample's option rows (at most n_opt of them)
    const long b0 = c.ooff ? c.ooff[n] : (long)n * NO, b1 = c.ooff ? c.ooff[n + 1] : b0 + NO;
    const int nq = (int)(b1 - b0);
    for (int i = threadIdx.x; i < nq; i += TB) {
        const int j = (int)(pt_onj(c, b0 + i) % NO);
        const float* oi = row + c.off.opt_int + (long)j * c.dm.opt_int;
        const int p1 = (int)oi[1], p2 = (int)oi[2];
        s_h1[i] = (p1 > 0 && p1 <= c.dm.l_tok) ? pt_hrow(c, n, p1) : -1;
        s_h2[i] = (p2 > 0 && p2 <= c.dm.l_tok) ? pt_hrow(c, n, p2) : -1;
        s_ty[i] = pt_id_clamp(oi[0], c.dm.n_opt_types - 1);
    }
    __syncthreads();
    constexpr int QB = 8;   // options whose gradient loads are issued together
    for (int col = threadIdx.x; col < D; col += TB) {
        for (int ib = 0; ib < nq; ib += QB) {
            float v1[QB], v2[QB];
#pragma unroll
            for (int u = 0; u < QB; ++u) {
                const int i = ib + u;
                v1[u] = v2[u] = 0.f;
                if (i >= nq) continue;
                const float* g = d_qin + (b0 + i) * W;
                if (s_h1[i] >= 0) v1[u] = g[PT_TYPE_E + col];
                if (s_h2[i] >= 0) v2[u] = g[PT_TYPE_E + D + col];
            }
#pragma unroll
            for (int u = 0; u < QB; ++u) {
                const int i = ib + u;
                if (i >= nq) break;
                if (v1[u] != 0.f) atomicAdd(d_h + s_h1[i] * D + col, v1[u]);
                if (v2[u] != 0.f) atomicAdd(d_h + s_h2[i] * D + col, v2[u]);
            }
        }
    }
    if (threadIdx.x < PT_TYPE_E) {
        IdCache k(d_temb, threadIdx.x);
        for (int i = 0; i < nq; ++i) k.add(s_ty[i], d_qin[(b0 + i) * W + threadIdx.x]);
        k.flush();
    }
}

// sc_in = [q (GEMM output) | r | g | dvec | q*r],  r = h[n,0], gd = [g | dvec]
__global__ void sc_in_fwd_kernel(GatherCtx c, const float* __restrict__ h,
        const float* __restrict__ gd, float* __restrict__ sc) {
    const int NO = c.dm.n_opt, D = c.dm.d, G = c.dm.g, W = c.dx.score_in;
    const int cw = W - D, ch = cw / 4;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= pt_orows(c) * ch) return;
    const int col = D + (int)(i % ch) * 4;
    const long row = i / ch;
    const int n = (int)(pt_onj(c, row) / NO);
    const float* r = h + pt_hrow(c, n, 0) * D;
    float* o = sc + row * W;
    float4 v;
    if (col < 2 * D) v = *reinterpret_cast<const float4*>(r + (col - D));
    else if (col < 2 * D + G + PT_DEC_H) v = *reinterpret_cast<const float4*>(gd + (long)n * c.dx.bcast_in + (col - 2 * D));
    else {
        const int e = col - (2 * D + G + PT_DEC_H);
        const float4 q = *reinterpret_cast<const float4*>(o + e);
        const float4 rr = *reinterpret_cast<const float4*>(r + e);
        v = make_float4(q.x * rr.x, q.y * rr.y, q.z * rr.z, q.w * rr.w);
    }
    *reinterpret_cast<float4*>(o + col) = v;
}

// one workgroup per sample: d_q = dsc[q] + dsc[qr]*r ; d_r, d_g, d_dvec summed
// over options.  SC_OG option groups of TB threads each sum a contiguous
// quarter of the options; the group partials add in a fixed order.
constexpr int SC_OG = 4;
__global__ __launch_bounds__(TB * SC_OG) void sc_in_bwd_kernel(GatherCtx c, const float* __restrict__ d_sc,
        const float* __restrict__ sc, float* __restrict__ d_q, float* __restrict__ d_h,
        float* __restrict__ d_gd) {
    extern __shared__ float red[];   // [3][SC_OG][span]
    const int n = blockIdx.x, NO = c.dm.n_opt, D = c.dm.d, G = c.dm.g, W = c.dx.score_in;
    const int o_r = D, o_g = 2 * D, o_dv = 2 * D + G, o_qr = 2 * D + G + PT_DEC_H;
    const int span = max(D, max(G, (int)PT_DEC_H));
    const int og = threadIdx.x / TB, t = threadIdx.x % TB;
    // the sample's option rows [b0, b0 + no), split into SC_OG contiguous groups
    const long b0 = c.ooff ? c.ooff[n] : (long)n * NO;
    const int no = c.ooff ? c.ooff[n + 1] - c.ooff[n] : NO;
    const int j0 = og * no / SC_OG, j1 = (og + 1) * no / SC_OG;
    for (int col = t; col < span; col += TB) {
        const float r = col < D ? sc[b0 * W + o_r + col] : 0.f;
        float ar = 0.f, ag = 0.f, adv = 0.f;
        for (int j = j0; j < j1; ++j) {
            const long nj = b0 + j;
            const float* g = d_sc + nj * W;
            if (col < D) {
                const float q = sc[nj * W + col];
                d_q[nj * D + col] = g[col] + g[o_qr + col] * r;
                ar += g[o_r + col] + g[o_qr + col] * q;
            }
            if (col < G) ag += g[o_g + col];
            if (col < PT_DEC_H) adv += g[o_dv + col];
        }
        red[(0 * SC_OG + og) * span + col] = ar;
        red[(1 * SC_OG + og) * span + col] = ag;
        red[(2 * SC_OG + og) * span + col] = adv;
    }
    __syncthreads();
    if (og != 0) return;
    for (int col = t; col < span; col += TB) {
        float ar = 0.f, ag = 0.f, adv = 0.f;
        for (int k = 0; k < SC_OG; ++k) {
            ar += red[(0 * SC_OG + k) * span + col];
            ag += red[(1 * SC_OG + k) * span + col];
            adv += red[(2 * SC_OG + k) * span + col];
        }
        if (col < D) d_h[pt_hrow(c, n, 0) * D + col] += ar;
        if (col < G) d_gd[(long)n * c.dx.bcast_in + col] += ag;
        if (col < PT_DEC_H) d_gd[(long)n * c.dx.bcast_in + G + col] += adv;
    }
}

__global__ void val_in_fwd_kernel(GatherCtx c, const float* __restrict__ h,
        const float* __restrict__ gd, float* __restrict__ v, int ls) {
    const int D = c.dm.d, W = c.dx.val_in;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)c.N * W) return;
    const int n = (int)(i / W), col = (int)(i % W);
    const long hr = ls == c.dx.l_seq ? pt_hrow(c, n, 0) : (long)n * ls;
    v[i] = col < D ? h[hr * D + col] : gd[(long)n * c.dx.bcast_in + (col - D)];
}

__global__ void val_in_bwd_kernel(GatherCtx c, const float* __restrict__ dv, float* __restrict__ d_h,
                                  float* __restrict__ d_gd, int ls) {
    const int D = c.dm.d, W = c.dx.val_in;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)c.N * W) return;
    const int n = (int)(i / W), col = (int)(i % W);
    const long hr = ls == c.dx.l_seq ? pt_hrow(c, n, 0) : (long)n * ls;
    if (col < D) d_h[hr * D + col] += dv[i];
    else d_gd[(long)n * c.dx.bcast_in + (col - D)] += dv[i];
}

// one wave per row: out = X[r,:] . w + b
// head rows: rmap (nullable) maps a row to its output / gradient slot q,
// rows_dev (nullable) bounds the rows on the device
__device__ __forceinline__ long hd_slot(const int* rmap, int r, int per, long ld, int col0) {
    const int q = rmap ? rmap[r] : r;
    return (long)(q / per) * ld + col0 + (q % per);
}

__global__ void head_dot_kernel(const float* __restrict__ X, int rows, int K,
        const float* __restrict__ w, const float* __restrict__ b, float* __restrict__ out, int per,
        long ldo, int col0, const int* __restrict__ rmap, const int* __restrict__ rows_dev) {
    if (rows_dev) rows = min(rows, *rows_dev);
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* x = X + (long)r * K;
    float s = 0.f;
    for (int k = lane; k < K; k += 64) s += x[k] * w[k];
    s = wave_sum(s);
    if (lane == 0) out[hd_slot(rmap, r, per, ldo, col0)] = s + b[0];
}

__global__ void head_dot_bwd_kernel(const float* __restrict__ grad, int per, long ldg, int col0,
        const float* __restrict__ w, const float* __restrict__ gd, float* __restrict__ dX, int rows,
        int K, const int* __restrict__ rmap, const int* __restrict__ rows_dev) {
    if (rows_dev) rows = min(rows, *rows_dev);
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)rows * K) return;
    const int r = (int)(i / K), k = (int)(i % K);
    const float dy = grad[hd_slot(rmap, r, per, ldg, col0)];
    dX[i] = dy * w[k] * gd[i];
}

constexpr int HD_ROWS = 64;
// partial[chunk][0..K) = sum dy*X, partial[chunk][K] = sum dy (every thread
// forms the dy sum alongside its column; thread 0 stores it)
__global__ void head_dot_dw_partial_kernel(const float* __restrict__ grad, int per, long ldg,
        int col0, const float* __restrict__ X, int rows, int K, float* __restrict__ part,
        const int* __restrict__ rmap, const int* __restrict__ rows_dev) {
    if (rows_dev) rows = min(rows, *rows_dev);
    const int r0 = blockIdx.x * HD_ROWS, r1 = min(rows, r0 + HD_ROWS);
    for (int k0 = 0; k0 < K; k0 += TB) {
        const int k = k0 + threadIdx.x;
        float s = 0.f, sd = 0.f;
        for (int rb = r0; rb < r1; rb += PF) {   // PF rows' loads together, sums in row order
            float dy[PF], xv[PF];
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                const int r = rb + u;
                dy[u] = r < r1 ? grad[hd_slot(rmap, r, per, ldg, col0)] : 0.f;
                xv[u] = (r < r1 && k < K) ? X[(long)r * K + k] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                if (rb + u >= r1) break;
                sd += dy[u];
                if (k < K) s += dy[u] * xv[u];
            }
        }
        if (k < K) part[(long)blockIdx.x * (K + 1) + k] = s;
        if (k0 == 0 && threadIdx.x == 0) part[(long)blockIdx.x * (K + 1) + K] = sd;
    }
}

// one workgroup per output column: strided chunk sums, then a fixed-order tree
__global__ void head_dot_dw_final_kernel(const float* __restrict__ part, int chunks, int K,
                                         float* __restrict__ dw, float* __restrict__ db) {
    __shared__ float red[TB];
    const int k = blockIdx.x;
    float s = 0.f;
    for (int ch = threadIdx.x; ch < chunks; ch += TB) s += part[(long)ch * (K + 1) + k];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = TB / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        if (k < K) dw[k] = red[0];
        else db[0] = red[0];
    }
}

__global__ void fill_zero_kernel(float4* p, long n4) {
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i < n4) p[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}
__global__ void fill_zero_tail_kernel(float* p, long n) {
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

#define PT_GRID(total) dim3(pt_cdiv((long)(total), TB)), dim3(TB), 0, s

}  // namespace

int pt_tok_cat_fwd(const GatherCtx& c, const float* card, const float* zemb, const float* oemb,
                   float* tok_cat, hipStream_t s, long rows_done) {
    PT_REQUIRE(c.dm.d_c % 4 == 0 && c.dm.tok_f % 4 == 0 && c.off.tok_float % 4 == 0 && c.stride % 4 == 0,
               "tok_cat: widths must be multiples of 4");
    const long rows = c.rowmap ? (long)c.N * c.dx.l_seq : (long)c.N * c.dm.l_tok;
    const int slot = pt_prof_open(s);
    hipLaunchKernelGGL(tok_cat_fwd_kernel, dim3(pt_cdiv(rows, TB / TOK_LPR)), dim3(TB), 0, s, c, card, zemb, oemb,
                       tok_cat);
    PT_LAUNCH_CHECK();
    // HBM bytes: each row written, its token's obs floats read (the embedding
    // tables, ~1 MB, stay in L2)
    pt_prof_close(slot, PROF_GATHER, (double)(rows_done > 0 ? rows_done : rows) * 4.0 *
                  (c.dx.tok_in + c.dm.tok_f + c.dm.tok_int), s);
    return PTCG_OK;
}
int pt_tok_cat_bwd(const GatherCtx& c, const float* d_cat, const DetSink& d_card, const DetSink& d_zemb,
                   const DetSink& d_oemb, hipStream_t s) {
    const long rows = c.rowmap ? (long)c.N * c.dx.l_seq : (long)c.N * c.dm.l_tok;
    const int cols = 2 * c.dm.d_c + PT_ZONE_E + PT_OWNER_E;
    PT_REQUIRE(cols <= 1024, "tok_cat_bwd: %d gradient columns", cols);
    hipLaunchKernelGGL(tok_cat_bwd_kernel, dim3(pt_cdiv(rows, SCATTER_ROWS)), dim3(pt_cdiv(cols, 64) * 64), 0, s, c,
                       d_cat, d_card, d_zemb, d_oemb);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_glob_in(const GatherCtx& c, float* glob_in, hipStream_t s) {
    hipLaunchKernelGGL(glob_in_kernel, PT_GRID((long)c.N * c.dm.global_f), c, glob_in);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_dec_in_fwd(const GatherCtx& c, const float* card, const float* att, const float* semb,
                  const float* cemb, float* dec_in, hipStream_t s) {
    hipLaunchKernelGGL(dec_in_fwd_kernel, PT_GRID((long)c.N * c.dx.dec_in), c, card, att, semb, cemb, dec_in);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_dec_in_bwd(const GatherCtx& c, const float* d_in, const DetSink& d_card, const DetSink& d_att,
                  const DetSink& d_semb, const DetSink& d_cemb, hipStream_t s) {
    hipLaunchKernelGGL(dec_in_bwd_kernel, dim3(pt_cdiv(c.dx.dec_in, TB), pt_cdiv(c.N, SCATTER_ROWS)), dim3(TB), 0, s,
                       c, d_in, d_card, d_att, d_semb, d_cemb);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_x0_fwd(const GatherCtx& c, const float* tokp, const float* bc, const float* readout, float* x0,
              float* keep, hipStream_t s, const float* lnw, const float* lnb, float* lny, float* lnmu, float* lnrs,
              int lnybf) {
    // one row per wave when the LayerNorm rides along (64 float4s per row, TB a multiple of 64)
    PT_REQUIRE(!lny || (c.dm.d == 256 && lnw && lnb && lnmu && lnrs), "x0 + layernorm: needs d = 256 and all buffers");
    hipLaunchKernelGGL(x0_fwd_kernel, PT_GRID((long)c.N * c.dx.l_seq * (c.dm.d / 4)), c, tokp, bc, readout, x0, keep,
                       lnw, lnb, lny, lnmu, lnrs, lnybf);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_x0_bwd(const GatherCtx& c, const float* d_x0, float* d_tokp, float* d_bc, hipStream_t s) {
    hipLaunchKernelGGL(x0_bwd_kernel, dim3(c.N), dim3(TB), 0, s, c, d_x0, d_tokp, d_bc);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_opt_gather_fwd(const GatherCtx& c, const float* card, const float* att, float* ocard, float* oatt,
                      hipStream_t s) {   // grids sized for all N * n_opt option rows
    const int W = c.dm.d_c > c.dm.d_a ? c.dm.d_c : c.dm.d_a;
    hipLaunchKernelGGL(opt_gather_fwd_kernel, PT_GRID((long)c.N * c.dm.n_opt * W), c, card, att, ocard, oatt);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_opt_gather_bwd(const GatherCtx& c, const float* d_ocard, const float* d_oatt, const DetSink& d_card,
                      const DetSink& d_att, hipStream_t s) {
    const int cols = c.dm.d_c + c.dm.d_a;
    PT_REQUIRE(cols <= 1024, "opt_gather_bwd: %d columns", cols);
    hipLaunchKernelGGL(opt_gather_bwd_kernel, dim3(pt_cdiv((long)c.N * c.dm.n_opt, SCATTER_ROWS)),
                       dim3(pt_cdiv(cols, 64) * 64), 0, s, c, d_ocard, d_oatt, d_card, d_att);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_q_in_fwd(const GatherCtx& c, const float* h, const float* temb, float* q_in, hipStream_t s) {
    PT_REQUIRE(c.dx.q_in % 4 == 0 && c.dm.opt_f % 4 == 0 && c.off.opt_float % 4 == 0, "q_in: widths must be multiples of 4");
    hipLaunchKernelGGL(q_in_fwd_kernel, PT_GRID((long)c.N * c.dm.n_opt * (c.dx.q_in / 4)), c, h, temb, q_in);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_q_in_bwd(const GatherCtx& c, const float* d_qin, float* d_h, const DetSink& d_temb, hipStream_t s) {
    PT_REQUIRE(c.dm.n_opt <= PT_MAX_OPT, "q_in backward: %d options per sample exceed %d", c.dm.n_opt, PT_MAX_OPT);
    hipLaunchKernelGGL(q_in_bwd_kernel, dim3(c.N), dim3(TB), 0, s, c, d_qin, d_h, d_temb);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_sc_in_fwd(const GatherCtx& c, const float* h, const float* gd, float* sc_in, hipStream_t s) {
    PT_REQUIRE(c.dm.g % 4 == 0, "sc_in: g must be a multiple of 4");
    hipLaunchKernelGGL(sc_in_fwd_kernel, PT_GRID((long)c.N * c.dm.n_opt * ((c.dx.score_in - c.dm.d) / 4)), c, h, gd, sc_in);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_sc_in_bwd(const GatherCtx& c, const float* d_sc, const float* sc_in, float* d_q, float* d_h,
                 float* d_gd, hipStream_t s) {
    const int span = std::max(c.dm.d, std::max(c.dm.g, (int)PT_DEC_H));
    hipLaunchKernelGGL(sc_in_bwd_kernel, dim3(c.N), dim3(TB * SC_OG), 3 * SC_OG * span * sizeof(float), s, c, d_sc,
                       sc_in, d_q, d_h, d_gd);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_val_in_fwd(const GatherCtx& c, const float* h, const float* gd, float* val_in, hipStream_t s, int ls) {
    hipLaunchKernelGGL(val_in_fwd_kernel, PT_GRID((long)c.N * c.dx.val_in), c, h, gd, val_in, ls ? ls : c.dx.l_seq);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_val_in_bwd(const GatherCtx& c, const float* d_val_in, float* d_h, float* d_gd, hipStream_t s, int ls) {
    hipLaunchKernelGGL(val_in_bwd_kernel, PT_GRID((long)c.N * c.dx.val_in), c, d_val_in, d_h, d_gd, ls ? ls : c.dx.l_seq);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_head_dot(const float* X, int rows, int K, const float* w, const float* b, float* out, int per,
                long ldo, int col0, hipStream_t s, const int* rmap, const int* rows_dev) {
    hipLaunchKernelGGL(head_dot_kernel, dim3(pt_cdiv(rows, 4)), dim3(256), 0, s, X, rows, K, w, b, out, per, ldo, col0,
                       rmap, rows_dev);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_head_dot_bwd(const float* grad, int per, long ldg, int col0, const float* w, const float* gd,
                    float* dX, int rows, int K, hipStream_t s, const int* rmap, const int* rows_dev) {
    hipLaunchKernelGGL(head_dot_bwd_kernel, PT_GRID((long)rows * K), grad, per, ldg, col0, w, gd, dX, rows, K, rmap,
                       rows_dev);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_head_dot_dw(const float* grad, int per, long ldg, int col0, const float* X, int rows, int K,
                   float* dw, float* db, float* ws, long ws_floats, hipStream_t s, const int* rmap,
                   const int* rows_dev) {
    const int chunks = pt_cdiv(rows, HD_ROWS);
    PT_REQUIRE(ws && (long)chunks * (K + 1) <= ws_floats, "head dw: workspace too small");
    hipLaunchKernelGGL(head_dot_dw_partial_kernel, dim3(chunks), dim3(TB), 0, s, grad, per, ldg, col0, X, rows, K, ws,
                       rmap, rows_dev);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(head_dot_dw_final_kernel, dim3(K + 1), dim3(TB), 0, s, ws, chunks, K, dw, db);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_fill_zero(float* p, long n, hipStream_t s) {
    if (n <= 0) return PTCG_OK;
    if (((uintptr_t)p & 15) == 0) {
        const long n4 = n / 4;
        if (n4) hipLaunchKernelGGL(fill_zero_kernel, PT_GRID(n4), (float4*)p, n4);
        if (n % 4) hipLaunchKernelGGL(fill_zero_tail_kernel, PT_GRID(n % 4), p + n4 * 4, n % 4);
    } else {
        hipLaunchKernelGGL(fill_zero_tail_kernel, PT_GRID(n), p, n);
    }
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
