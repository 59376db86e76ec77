// Kernels of the reference model variant: the static-table chain, the
// oracle critic's input and output plumbing, and the belief / blind-value
// aux losses the backward injects.
//
// Reference counterparts (native/model/ptcg_model.cu, ptcg_model2.cu,
// ptcg_model3.cu):
//   k_pool :236 / k_pool_bwd :15                 -> pool_fwd / pool_bwd
//   k_att_in :218, k_sk_in :229, k_card_in :260  -> column copies into
//       concat buffers whose static / text columns are filled once at upload
//   k_otok_in :441 / k_otok_bwd :159             -> otok_in_fwd / otok_bwd
//   k_xc :484 / k_xc_bwd :177                    -> xc_fwd / xc_bwd
//   k_aux_targets :220, k_hand_grad :237, k_prize_count :245,
//   k_prize_grad :263, k_blind_grad :281         -> aux_count + aux_rows
//   k_prize_head / k_prize_head_bwd (ptcg_model3.cu:411-438) -> head_dot +
//       rank1_add
// Shared-table scatters (card rows referenced by several cards / tokens /
// options), where the reference uses fp32 atomics, add in 64-bit fixed point
// (detsum.hip), so their sums do not depend on the order the adds land in;
// per-sample work runs one workgroup per sample with the targets built in LDS.
#include "model.h"

namespace {

constexpr int TB = 256;
#define FZ_GRID(total) dim3(pt_cdiv((long)(total), TB)), dim3(TB), 0, s

__device__ __forceinline__ int obs_id(float v) { return (int)v; }   // C truncation toward zero
__device__ __forceinline__ int clamp_id(int id, int n) { return id < 0 ? 0 : (id >= n ? n - 1 : id); }

__global__ void fill_int_zero_kernel(int* p, int n) {
    if ((int)threadIdx.x < n) p[threadIdx.x] = 0;
}

__global__ void copy_cols_kernel(float* __restrict__ dst, long ldd, const float* __restrict__ src, long lds,
                                 int rows, int cols) {
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i % cols);
    dst[(long)r * ldd + c] = src[(long)r * lds + c];
}

// masked mean / max over the K table rows a card lists (id 0 = empty slot);
// empty slots take part in the max as 0; amax = first maximal slot.
__global__ void pool_fwd_kernel(const float* __restrict__ tab, int E, const int* __restrict__ ids, int K,
                                int NC, float* __restrict__ out, long ldo, int col_mean, int col_max,
                                int* __restrict__ amax) {
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)NC * E) return;
    const int n = (int)(i / E), e = (int)(i % E);
    float s = 0.f, mx = -1e30f;
    int cnt = 0, am = 0;
    for (int k = 0; k < K; ++k) {
        const int id = ids[n * K + k];
        const float v = id > 0 ? tab[(long)id * E + e] : 0.f;
        if (id > 0) { ++cnt; s += v; }
        if (v > mx) { mx = v; am = k; }
    }
    out[(long)n * ldo + col_mean + e] = s / (float)(cnt > 0 ? cnt : 1);
    out[(long)n * ldo + col_max + e] = mx;
    amax[i] = am;
}

__global__ void pool_bwd_kernel(const float* __restrict__ dsrc, long ld, int col_mean, int col_max,
                                const int* __restrict__ amax, const int* __restrict__ ids, int K, int NC,
                                int E, DetSink d_tab) {
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)NC * E) return;
    const int n = (int)(i / E), e = (int)(i % E);
    int cnt = 0;
    for (int k = 0; k < K; ++k) cnt += ids[n * K + k] > 0 ? 1 : 0;
    const float dm = dsrc[(long)n * ld + col_mean + e] / (float)(cnt > 0 ? cnt : 1);
    const float dx = dsrc[(long)n * ld + col_max + e];
    const int am = amax[i];
    const double sc = *d_tab.scale;
    for (int k = 0; k < K; ++k) {
        const int id = ids[n * K + k];
        if (id <= 0) continue;
        pt_det_add(d_tab, sc, (long)id * E + e, dm + (k == am ? dx : 0.f));
    }
}

__global__ void mul_kernel(const float* __restrict__ dy, const float* __restrict__ gd,
                           float* __restrict__ dx, long n) {
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i < n) dx[i] = dy[i] * gd[i];
}

// oracle token inputs (N, n_orc, d_c + 6) = [CardVec(id) | kind one-hot 3 |
// count | deck | prize], and the critic key mask [1 | trunk keep | id > 0].
__global__ void otok_in_kernel(GatherCtx c, const float* __restrict__ cv, const float* __restrict__ keep,
                               float* __restrict__ out, float* __restrict__ ckeep) {
    const int DC = c.dm.d_c, W = c.dx.orc_in, NO = c.dx.n_orc, Ls = c.dx.l_seq;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)c.N * NO * W) return;
    const int col = (int)(i % W);
    const long nk = i / W;
    const int k = (int)(nk % NO), n = (int)(nk / NO);
    const float* o = obs_row(c.obs, c.idx, c.stride, n) + c.off.oracle;
    int id, kind;
    float f3 = 0.f, f4 = 0.f, f5 = 0.f;
    if (k < PT_N_HAND) {
        kind = 0; id = obs_id(o[2 * k]); f3 = o[2 * k + 1];
    } else if (k < PT_N_HAND + PT_N_SPLIT) {
        const int sl = k - PT_N_HAND;
        const float* so = o + 2 * PT_N_HAND + 3 * sl;
        kind = 1; id = obs_id(so[0]); f4 = so[1]; f5 = so[2];
    } else {
        const int sl = k - PT_N_HAND - PT_N_SPLIT;
        const float* po = o + 2 * PT_N_HAND + 3 * PT_N_SPLIT + 2 * sl;
        kind = 2; id = obs_id(po[0]); f3 = po[1];
    }
    const int idc = clamp_id(id, c.dm.n_cards);
    float v;
    if (col < DC) v = cv[(long)idc * DC + col];
    else if (col < DC + 3) v = (col - DC) == kind ? 1.f : 0.f;
    else if (col == DC + 3) v = f3;
    else if (col == DC + 4) v = f4;
    else v = f5;
    out[i] = v;
    if (col == 0) {
        float* ck = ckeep + (long)n * c.dx.l_crit;
        if (k == 0) {
            ck[0] = 1.f;
            for (int l = 0; l < Ls; ++l) ck[1 + l] = keep[(long)n * Ls + l];
        }
        ck[1 + Ls + k] = id > 0 ? 1.f : 0.f;
    }
}

__global__ void otok_bwd_kernel(GatherCtx c, const float* __restrict__ d_in, DetSink d_card) {
    const int DC = c.dm.d_c, W = c.dx.orc_in, NO = c.dx.n_orc;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)c.N * NO * DC) return;
    const int col = (int)(i % DC);
    const long nk = i / DC;
    const int k = (int)(nk % NO), n = (int)(nk / NO);
    const float g = d_in[nk * W + col];
    if (g == 0.f) return;
    const float* o = obs_row(c.obs, c.idx, c.stride, n) + c.off.oracle;
    const int id = k < PT_N_HAND ? obs_id(o[2 * k])
                 : k < PT_N_HAND + PT_N_SPLIT ? obs_id(o[2 * PT_N_HAND + 3 * (k - PT_N_HAND)])
                 : obs_id(o[2 * PT_N_HAND + 3 * PT_N_SPLIT + 2 * (k - PT_N_HAND - PT_N_SPLIT)]);
    pt_det_add(d_card, *d_card.scale, (long)clamp_id(id, c.dm.n_cards) * DC + col, g);
}

// critic sequence (N, l_crit, D) = [critic readout | h (l_seq rows) | otok]
__global__ void xc_fwd_kernel(const float* __restrict__ cread, const float* __restrict__ h,
                              const float* __restrict__ otok, float* __restrict__ xc, int N, int Ls, int NO,
                              int D) {
    const int Lc = 1 + Ls + NO;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)N * Lc * D) return;
    const int d = (int)(i % D);
    const long nl = i / D;
    const int l = (int)(nl % Lc), n = (int)(nl / Lc);
    float v;
    if (l == 0) v = cread[d];
    else if (l <= Ls) v = h[((long)n * Ls + (l - 1)) * D + d];
    else v = otok[((long)n * NO + (l - 1 - Ls)) * D + d];
    xc[i] = v;
}

// d_h += d_xc[:, 1..Ls], d_otok = d_xc[:, Ls+1..]  (the readout row is column-summed)
__global__ void xc_bwd_kernel(const float* __restrict__ d_xc, float* __restrict__ d_h, float* __restrict__ d_otok,
                              int N, int Ls, int NO, int D) {
    const int Lc = 1 + Ls + NO;
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)N * (Lc - 1) * D) return;
    const int d = (int)(i % D);
    const long nl = i / D;
    const int l = 1 + (int)(nl % (Lc - 1)), n = (int)(nl / (Lc - 1));
    const float g = d_xc[((long)n * Lc + l) * D + d];
    if (l <= Ls) d_h[((long)n * Ls + (l - 1)) * D + d] += g;
    else d_otok[((long)n * NO + (l - 1 - Ls)) * D + d] = g;
}

// number of MY_UNSEEN tokens in the minibatch (the prize loss normaliser)
__global__ void aux_count_kernel(GatherCtx c, int* __restrict__ cnt) {
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    int v = 0;
    if (i < (long)c.N * c.dm.l_tok) {
        const int n = (int)(i / c.dm.l_tok), l = (int)(i % c.dm.l_tok);
        const float* ti = obs_row(c.obs, c.idx, c.stride, n) + c.off.tok_int + (long)l * c.dm.tok_int;
        v = obs_id(ti[1]) == PT_ZONE_MY_UNSEEN ? 1 : 0;
    }
    v = (int)wave_sum((float)v);   // <= 64, exact in fp32
    if ((threadIdx.x & 63) == 0 && v) atomicAdd(cnt, v);
}

__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }

// One workgroup per sample: opp-hand count targets and my-prize indicators
// in LDS, then
//   d_hand[n][j]  = 0.1 * 2 (softplus(x) - t) / (N * NC) * sigmoid(x)  (x > 20: 1)
//   d_prize[n][l] = 0.1 (sigmoid(logit) - prized[cid]) / count on MY_UNSEEN tokens
//   d_blind[n]    = (v - return) / N
// d_prize has the (N, l_seq) layout of the prize head's output (column 0,
// the READOUT row, gets 0).
__global__ void aux_rows_kernel(GatherCtx c, const float* __restrict__ hand_lin,
                                const float* __restrict__ prize_all, const float* __restrict__ blind_v,
                                const float* __restrict__ ret, const int* __restrict__ cnt,
                                float* __restrict__ d_hand, float* __restrict__ d_prize,
                                float* __restrict__ d_blind) {
    extern __shared__ float sh[];
    const int NC = c.dm.n_cards, Ls = c.dx.l_seq, N = c.N;
    float* tgt = sh;
    float* prized = sh + NC;
    const int n = blockIdx.x;
    const float* row = obs_row(c.obs, c.idx, c.stride, n);
    const float* o = row + c.off.oracle;
    for (int j = threadIdx.x; j < 2 * NC; j += blockDim.x) sh[j] = 0.f;
    __syncthreads();
    if (threadIdx.x == 0) {   // slot order, as the reference's per-slot adds
        for (int k = 0; k < PT_N_HAND; ++k) {
            const int id = obs_id(o[2 * k]);
            const float cn = o[2 * k + 1] * 4.0f;
            if (id > 0 && id < NC && id != NC - 1 && cn != 0.f) tgt[id] += cn;
        }
        const float* po = o + 2 * PT_N_HAND + 3 * PT_N_SPLIT;
        for (int k = 0; k < PT_N_PRIZE; ++k) {
            const int id = obs_id(po[2 * k]);
            if (id > 0 && id < NC && po[2 * k + 1] > 0.f) prized[id] = 1.f;
        }
    }
    __syncthreads();
    const float hs = PT_AUX_HAND * 2.f / ((float)N * (float)NC);
    for (int j = threadIdx.x; j < NC; j += blockDim.x) {
        const float x = hand_lin[(long)n * NC + j];
        const float g = hs * (softplus_f(x) - tgt[j]);
        d_hand[(long)n * NC + j] = x > 20.f ? g : g * sigmoid_f(x);
    }
    const float cc = (float)(cnt[0] > 0 ? cnt[0] : 1);
    for (int l = threadIdx.x; l < Ls; l += blockDim.x) {
        float g = 0.f;
        if (l > 0) {
            const float* ti = row + c.off.tok_int + (long)(l - 1) * c.dm.tok_int;
            if (obs_id(ti[1]) == PT_ZONE_MY_UNSEEN) {
                const float t = prized[clamp_id(obs_id(ti[0]), NC)];
                g = PT_AUX_PRIZE * (sigmoid_f(prize_all[(long)n * Ls + l]) - t) / cc;
            }
        }
        d_prize[(long)n * Ls + l] = g;
    }
    if (threadIdx.x == 0) {
        const long r = c.idx ? (long)c.idx[n] : (long)n;
        d_blind[n] = PT_AUX_VF * (blind_v[n] - ret[r]) / (float)N;
    }
}

// dX[r, :] += dy[r] * w[:]
__global__ void rank1_add_kernel(const float* __restrict__ dy, const float* __restrict__ w,
                                 float* __restrict__ dX, int rows, int K) {
    const long i = (long)blockIdx.x * TB + threadIdx.x;
    if (i >= (long)rows * K) return;
    const int r = (int)(i / K), k = (int)(i % K);
    const float g = dy[r];
    if (g != 0.f) dX[i] += g * w[k];
}

}  // namespace

int pt_copy_cols(float* dst, long ldd, const float* src, long lds, int rows, int cols, hipStream_t s) {
    hipLaunchKernelGGL(copy_cols_kernel, FZ_GRID((long)rows * cols), dst, ldd, src, lds, rows, cols);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_pool_fwd(const float* tab, int E, const int* ids, int K, int NC, float* out, long ldo, int col_mean,
                int col_max, int* amax, hipStream_t s) {
    hipLaunchKernelGGL(pool_fwd_kernel, FZ_GRID((long)NC * E), tab, E, ids, K, NC, out, ldo, col_mean, col_max, amax);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_pool_bwd(const float* dsrc, long ld, int col_mean, int col_max, const int* amax, const int* ids, int K,
                int NC, int E, const DetSink& d_tab, hipStream_t s) {
    hipLaunchKernelGGL(pool_bwd_kernel, FZ_GRID((long)NC * E), dsrc, ld, col_mean, col_max, amax, ids, K, NC, E, d_tab);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_mul(const float* dy, const float* gd, float* dx, long n, hipStream_t s) {
    hipLaunchKernelGGL(mul_kernel, FZ_GRID(n), dy, gd, dx, n);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_otok_in(const GatherCtx& c, const float* cv, const float* keep, float* out, float* ckeep, hipStream_t s) {
    hipLaunchKernelGGL(otok_in_kernel, FZ_GRID((long)c.N * c.dx.n_orc * c.dx.orc_in), c, cv, keep, out, ckeep);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_otok_bwd(const GatherCtx& c, const float* d_in, const DetSink& d_card, hipStream_t s) {
    hipLaunchKernelGGL(otok_bwd_kernel, FZ_GRID((long)c.N * c.dx.n_orc * c.dm.d_c), c, d_in, d_card);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_xc_fwd(const float* cread, const float* h, const float* otok, float* xc, int N, int Ls, int NO, int D,
              hipStream_t s) {
    hipLaunchKernelGGL(xc_fwd_kernel, FZ_GRID((long)N * (1 + Ls + NO) * D), cread, h, otok, xc, N, Ls, NO, D);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_xc_bwd(const float* d_xc, float* d_h, float* d_otok, int N, int Ls, int NO, int D, hipStream_t s) {
    hipLaunchKernelGGL(xc_bwd_kernel, FZ_GRID((long)N * (Ls + NO) * D), d_xc, d_h, d_otok, N, Ls, NO, D);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_aux_grads(const GatherCtx& c, const float* hand_lin, const float* prize_all, const float* blind_v,
                 const float* ret, int* cnt, float* d_hand, float* d_prize, float* d_blind, hipStream_t s) {
    PT_REQUIRE(ret != nullptr, "aux losses: returns not bound (ptcg_model_bind_returns)");
    hipLaunchKernelGGL(fill_int_zero_kernel, dim3(1), dim3(64), 0, s, cnt, 1);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(aux_count_kernel, FZ_GRID((long)c.N * c.dm.l_tok), c, cnt);
    PT_LAUNCH_CHECK();
    const size_t lds = 2 * (size_t)c.dm.n_cards * sizeof(float);
    PT_REQUIRE(lds <= 64 * 1024, "aux losses: n_cards=%d too large", c.dm.n_cards);
    hipLaunchKernelGGL(aux_rows_kernel, dim3(c.N), dim3(TB), lds, s, c, hand_lin, prize_all, blind_v, ret, cnt,
                       d_hand, d_prize, d_blind);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
int pt_rank1_add(const float* dy, const float* w, float* dX, int rows, int K, hipStream_t s) {
    hipLaunchKernelGGL(rank1_add_kernel, FZ_GRID((long)rows * K), dy, w, dX, rows, K);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
