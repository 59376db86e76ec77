// Masked multi-head self-attention over padded entity tokens, fused per
// (sample, head), fp32.
//
// Replaces the reference's chain pt_qkv_split -> batched QK^T GEMM ->
// pt_attn_softmax_fwd -> batched PV GEMM -> pt_heads_merge and its backward
// (native/model/ptcg_kernels.cuh:223-348, ptcg_model3.cu:18-30,63-91), which
// materialises the (N,H,L,L) probabilities in HBM per layer.  Here one
// workgroup owns one (sample, head): Q, K, V for that head are read straight
// out of the (N, L, 3D) qkv rows into LDS, the softmax row lives in LDS, and
// only the context rows (written into the merged (N, L, D) layout at column
// h*Dh) and one log-sum-exp per query row leave the chip.  The backward
// recomputes P from Q, K and the saved log-sum-exp.
//
// Semantics (ptcg_kernels.cuh:223-289): scores * (1/sqrt(Dh)); keys with
// keep == 0 score -1e30 (so they get probability exactly 0); the READOUT key
// is always kept, so no row is fully masked.  dS = P o (dP - rowsum(dO o O)).
#include "common.h"

namespace {

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------------------ forward
// LDS: Qs[L][DH+1], Ks[L][DH+1], Vs[L][DH], Pw[4][64*KPL], kf[L]
template <int DH, int KPL>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const float* __restrict__ qkv,
        const float* __restrict__ keep, float* __restrict__ ctx, float* __restrict__ lse,
        int L, int H, float scale) {
    extern __shared__ float sm[];
    constexpr int SQ = DH + 1;
    float* Qs = sm;
    float* Ks = Qs + L * SQ;
    float* Vs = Ks + L * SQ;
    float* Pw = Vs + L * DH;
    float* kf = Pw + 4 * 64 * KPL;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = blockIdx.x / H, h = blockIdx.x % H;
    const int D = H * DH;
    const float* base = qkv + (long)n * L * 3 * D + h * DH;
    for (int idx = tid; idx < L * DH; idx += 256) {
        const int l = idx / DH, d = idx % DH;
        const float* r = base + (long)l * 3 * D + d;
        Qs[l * SQ + d] = r[0];
        Ks[l * SQ + d] = r[D];
        Vs[l * DH + d] = r[2 * D];
    }
    for (int l = tid; l < L; l += 256) kf[l] = keep[(long)n * L + l];
    __syncthreads();

    float* P = Pw + wave * 64 * KPL;
    constexpr int RPW = 64 / DH;           // query rows handled per wave pass in the PV step
    const int sub = lane / DH, d = lane % DH;
    for (int i = wave; i < L; i += 4) {
        const float* q = Qs + i * SQ;
        float s[KPL];
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < KPL; ++c) {
            const int j = lane + 64 * c;
            s[c] = -INFINITY;
            if (j < L) {
                const float* k = Ks + j * SQ;
                float acc = 0.f;
#pragma unroll 16
                for (int e = 0; e < DH; ++e) acc += q[e] * k[e];
                s[c] = kf[j] != 0.f ? acc * scale : -1e30f;
            }
            mx = fmaxf(mx, s[c]);
        }
        mx = wave_max(mx);
        float sum = 0.f;
#pragma unroll
        for (int c = 0; c < KPL; ++c) {
            const int j = lane + 64 * c;
            float e = j < L ? expf(s[c] - mx) : 0.f;
            s[c] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        const float inv = 1.0f / sum;
#pragma unroll
        for (int c = 0; c < KPL; ++c) P[lane + 64 * c] = s[c] * inv;
        if (lane == 0) lse[((long)n * H + h) * L + i] = mx + logf(sum);
        wave_lds_sync();
        float o = 0.f;
        for (int j = sub; j < L; j += RPW) o += P[j] * Vs[j * DH + d];
        if (RPW == 2) o += __shfl_xor(o, 32, 64);
        if (sub == 0) ctx[((long)n * L + i) * D + h * DH + d] = o;
        wave_lds_sync();
    }
}

// ------------------------------------------------------------------ backward
// LDS: Qs, Ks, Vs, dOs [L][DH+1]; Pm[L][L+1]; Dv[L]; ls[L]; kf[L]
template <int DH, int KPL>
__global__ __launch_bounds__(256) void attn_bwd_kernel(const float* __restrict__ qkv,
        const float* __restrict__ keep, const float* __restrict__ ctx,
        const float* __restrict__ lse, const float* __restrict__ dctx,
        float* __restrict__ dqkv, int L, int H, float scale) {
    extern __shared__ float sm[];
    constexpr int SQ = DH + 1;
    const int SP = L + 1;
    float* Qs = sm;
    float* Ks = Qs + L * SQ;
    float* Vs = Ks + L * SQ;
    float* dOs = Vs + L * SQ;
    float* Pm = dOs + L * SQ;
    float* Dv = Pm + L * SP;
    float* ls = Dv + L;
    float* kf = ls + L;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = blockIdx.x / H, h = blockIdx.x % H;
    const int D = H * DH;
    const float* base = qkv + (long)n * L * 3 * D + h * DH;
    const float* ob = ctx + (long)n * L * D + h * DH;
    const float* dob = dctx + (long)n * L * D + h * DH;
    float* gb = dqkv + (long)n * L * 3 * D + h * DH;
    for (int idx = tid; idx < L * DH; idx += 256) {
        const int l = idx / DH, d = idx % DH;
        const float* r = base + (long)l * 3 * D + d;
        Qs[l * SQ + d] = r[0];
        Ks[l * SQ + d] = r[D];
        Vs[l * SQ + d] = r[2 * D];
        dOs[l * SQ + d] = dob[(long)l * D + d];
    }
    for (int l = tid; l < L; l += 256) {
        kf[l] = keep[(long)n * L + l];
        ls[l] = lse[((long)n * H + h) * L + l];
    }
    // Dv[i] = sum_d dO[i][d] * O[i][d]   (one wave per row)
    constexpr int RPW = 64 / DH;
    const int sub = lane / DH, d = lane % DH;
    for (int i = wave; i < L; i += 4) {
        float v = (sub == 0) ? dob[(long)i * D + d] * ob[(long)i * D + d] : 0.f;
        v = wave_sum(v);
        if (lane == 0) Dv[i] = v;
    }
    __syncthreads();

    // phase 1: P[i][j] = exp(s_ij*scale - lse_i) on kept keys
    for (int i = wave; i < L; i += 4) {
        const float* q = Qs + i * SQ;
        const float li = ls[i];
#pragma unroll
        for (int c = 0; c < KPL; ++c) {
            const int j = lane + 64 * c;
            if (j < L) {
                const float* k = Ks + j * SQ;
                float acc = 0.f;
#pragma unroll 16
                for (int e = 0; e < DH; ++e) acc += q[e] * k[e];
                Pm[i * SP + j] = kf[j] != 0.f ? expf(acc * scale - li) : 0.f;
            }
        }
    }
    __syncthreads();

    // phase 2: dV[j] = sum_i P[i][j] dO[i]
    for (int j0 = wave * RPW; j0 < L; j0 += 4 * RPW) {
        const int j = j0 + sub;
        if (j < L) {
            float acc = 0.f;
            for (int i = 0; i < L; ++i) acc += Pm[i * SP + j] * dOs[i * SQ + d];
            gb[(long)j * 3 * D + 2 * D + d] = acc;
        }
    }
    __syncthreads();

    // phase 3: dS[i][j] = P (dP - Dv_i), dP = dO_i . V_j ; dQ_i = scale * sum_j dS_ij K_j
    for (int i = wave; i < L; i += 4) {
        const float* dor = dOs + i * SQ;
        const float di = Dv[i];
#pragma unroll
        for (int c = 0; c < KPL; ++c) {
            const int j = lane + 64 * c;
            if (j < L) {
                const float* v = Vs + j * SQ;
                float acc = 0.f;
#pragma unroll 16
                for (int e = 0; e < DH; ++e) acc += dor[e] * v[e];
                Pm[i * SP + j] = Pm[i * SP + j] * (acc - di);
            }
        }
        wave_lds_sync();
        float acc = 0.f;
        for (int j = sub; j < L; j += RPW) acc += Pm[i * SP + j] * Ks[j * SQ + d];
        if (RPW == 2) acc += __shfl_xor(acc, 32, 64);
        if (sub == 0) gb[(long)i * 3 * D + d] = acc * scale;
        wave_lds_sync();
    }
    __syncthreads();

    // phase 4: dK[j] = scale * sum_i dS[i][j] Q[i]
    for (int j0 = wave * RPW; j0 < L; j0 += 4 * RPW) {
        const int j = j0 + sub;
        if (j < L) {
            float acc = 0.f;
            for (int i = 0; i < L; ++i) acc += Pm[i * SP + j] * Qs[i * SQ + d];
            gb[(long)j * 3 * D + D + d] = acc * scale;
        }
    }
}

// ======================================================= MFMA (fp32) path
// v_mfma_f32_16x16x4_f32 lane layout: A[i][k] from lane i + 16k, B[k][j] from
// lane j + 16k, D[i][j] in lane j + 16(i/4), register i%4.  A score tile
// computed as D = K Q^T holds key 16J + 4g + r of query li in lane (li, g),
// register r; feeding register r of every lane as the A operand of the next
// MFMA reduces over keys {16J + 4g + r : g = 0..3} — a permutation of the
// key dimension — so P goes from accumulators to the P.V product without
// touching LDS (B supplies V rows in the same key order).  The padded length
// Lp = 16 * ceil(L / 16); padded keys score -inf, padded rows are zero.
// 8 waves per workgroup: one 16-row stripe each (Lp <= 128), two waves per
// SIMD to overlap LDS reads with MFMAs.

template <int DH, int NT>   // NT = Lp / 16 key (and query) tiles
__global__ __launch_bounds__(512) void attn_fwd_mfma_kernel(const float* __restrict__ qkv,
        const float* __restrict__ keep, float* __restrict__ ctx, float* __restrict__ lse,
        int L, int H, float scale) {
    constexpr int LP = NT * 16, SK = DH + 4;
    __shared__ float Ks[LP * SK];
    __shared__ float Vs[LP * SK];
    __shared__ float kf[LP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int n = blockIdx.x / H, h = blockIdx.x % H;
    const int D = H * DH;
    const gfloat* base = (const gfloat*)qkv + (long)n * L * 3 * D + h * DH;
    for (int idx = tid; idx < LP * (DH / 4); idx += 512) {
        const int l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
        float4 k4 = make_float4(0.f, 0.f, 0.f, 0.f), v4 = k4;
        if (l < L) {
            const gfloat* r = base + (long)l * 3 * D + c4;
            k4 = ld_g4(r + D);
            v4 = ld_g4(r + 2 * D);
        }
        *reinterpret_cast<float4*>(&Ks[l * SK + c4]) = k4;
        *reinterpret_cast<float4*>(&Vs[l * SK + c4]) = v4;
    }
    for (int l = tid; l < LP; l += 512) kf[l] = l < L ? (keep[(long)n * L + l] != 0.f ? 1.f : 0.f) : -1.f;
    __syncthreads();

    for (int st = wave; st < NT; st += 8) {
        const int q0 = st * 16;
        // Q^T as the B operand: lane (li = query, lq) holds Q[q0+li][4kk+lq]
        float qb[DH / 4];
        const bool qv = q0 + li < L;
#pragma unroll
        for (int kk = 0; kk < DH / 4; ++kk)
            qb[kk] = qv ? base[(long)(q0 + li) * 3 * D + 4 * kk + lq] : 0.f;
        floatx4 sc[NT];
#pragma unroll
        for (int J = 0; J < NT; ++J) {
            sc[J] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < DH / 4; ++kk)
                sc[J] = __builtin_amdgcn_mfma_f32_16x16x4f32(Ks[(16 * J + li) * SK + 4 * kk + lq], qb[kk], sc[J], 0, 0, 0);
        }
        // sc[J][r] = S^T[key = 16J + 4lq + r][query = q0 + li]
        float mx = -INFINITY;
#pragma unroll
        for (int J = 0; J < NT; ++J)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float f = kf[16 * J + 4 * lq + r];
                const float v = f > 0.f ? sc[J][r] * scale : (f == 0.f ? -1e30f : -INFINITY);
                sc[J][r] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        float sum = 0.f;
#pragma unroll
        for (int J = 0; J < NT; ++J)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = expf(sc[J][r] - mx);
                sc[J][r] = e;
                sum += e;
            }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        // O = P V over the permuted key order
        floatx4 o[DH / 16];
#pragma unroll
        for (int dt = 0; dt < DH / 16; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int J = 0; J < NT; ++J)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float* vr = &Vs[(16 * J + 4 * lq + r) * SK + li];
#pragma unroll
                for (int dt = 0; dt < DH / 16; ++dt)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sc[J][r], vr[16 * dt], o[dt], 0, 0, 0);
            }
        // o[dt][r] = O[q0 + 4lq + r][16dt + li] * sum(query); normalise
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float inv = 1.0f / __shfl(sum, 4 * lq + r, 64);
            const int q = q0 + 4 * lq + r;
            if (q < L) {
                gfloat* dst = (gfloat*)ctx + ((long)n * L + q) * D + h * DH + li;
#pragma unroll
                for (int dt = 0; dt < DH / 16; ++dt) dst[16 * dt] = o[dt][r] * inv;
            }
        }
        if (lq == 0 && qv) lse[((long)n * H + h) * L + q0 + li] = mx + logf(sum);
    }
}

// Backward.  Pass A walks key stripes: per query tile it recomputes
// S = Q K^T and dP = dO V^T with keys on lanes, forms P and
// dS = P (dP - rowsum(dO o O)), accumulates dV += P^T dO and dK += dS^T Q
// (register-r trick again, now over queries), and parks dS*scale in LDS.
// Pass B walks query stripes: dQ = dS K from LDS.
template <int DH, int NT>
__global__ __launch_bounds__(512) void attn_bwd_mfma_kernel(const float* __restrict__ qkv,
        const float* __restrict__ keep, const float* __restrict__ ctx,
        const float* __restrict__ lse, const float* __restrict__ dctx,
        float* __restrict__ dqkv, int L, int H, float scale) {
    constexpr int LP = NT * 16, SQ = DH + 4, SKB = DH + 16, SS = LP + 4;
    extern __shared__ float sm[];
    float* Qs = sm;                 // [LP][SQ]
    float* dOs = Qs + LP * SQ;      // [LP][SQ]
    float* Ks = dOs + LP * SQ;      // [LP][SKB]
    float* dSs = Ks + LP * SKB;     // [LP][SS]  (query-major)
    float* ls = dSs + LP * SS;      // [LP]
    float* Dv = ls + LP;            // [LP]
    float* kf = Dv + LP;            // [LP]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int n = blockIdx.x / H, h = blockIdx.x % H;
    const int D = H * DH;
    const gfloat* base = (const gfloat*)qkv + (long)n * L * 3 * D + h * DH;
    const gfloat* ob = (const gfloat*)ctx + (long)n * L * D + h * DH;
    const gfloat* dob = (const gfloat*)dctx + (long)n * L * D + h * DH;
    gfloat* gb = (gfloat*)dqkv + (long)n * L * 3 * D + h * DH;
    for (int idx = tid; idx < LP * (DH / 4); idx += 512) {
        const int l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
        float4 q4 = make_float4(0.f, 0.f, 0.f, 0.f), k4 = q4, d4 = q4;
        if (l < L) {
            const gfloat* r = base + (long)l * 3 * D + c4;
            q4 = ld_g4(r);
            k4 = ld_g4(r + D);
            d4 = ld_g4(dob + (long)l * D + c4);
        }
        *reinterpret_cast<float4*>(&Qs[l * SQ + c4]) = q4;
        *reinterpret_cast<float4*>(&dOs[l * SQ + c4]) = d4;
        *reinterpret_cast<float4*>(&Ks[l * SKB + c4]) = k4;
    }
    for (int l = tid; l < LP; l += 512) {
        kf[l] = l < L ? (keep[(long)n * L + l] != 0.f ? 1.f : 0.f) : 0.f;
        ls[l] = l < L ? lse[((long)n * H + h) * L + l] : INFINITY;
    }
    // Dv[q] = sum_d dO[q][d] O[q][d]   (a wave per row; padded rows 0)
    for (int q = wave; q < LP; q += 8) {
        float v = 0.f;
        if (q < L)
            for (int d = lane; d < DH; d += 64) v += dob[(long)q * D + d] * ob[(long)q * D + d];
        v = wave_sum(v);
        if (lane == 0) Dv[q] = v;
    }
    __syncthreads();

    // ---- pass A: key stripes
    for (int kb = wave; kb < NT; kb += 8) {
        const int k0 = kb * 16;
        const bool kv = k0 + li < L;
        float kr[DH / 4], vr[DH / 4];    // B operands: lane (li = key, lq) holds K/V[k0+li][4kk+lq]
#pragma unroll
        for (int kk = 0; kk < DH / 4; ++kk) {
            kr[kk] = kv ? base[(long)(k0 + li) * 3 * D + D + 4 * kk + lq] : 0.f;
            vr[kk] = kv ? base[(long)(k0 + li) * 3 * D + 2 * D + 4 * kk + lq] : 0.f;
        }
        const float kfl = kf[k0 + li];
        floatx4 dv[DH / 16], dk[DH / 16];
#pragma unroll
        for (int dt = 0; dt < DH / 16; ++dt) {
            dv[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
            dk[dt] = dv[dt];
        }
        for (int qt = 0; qt < NT; ++qt) {
            floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f}, dp = s;
#pragma unroll
            for (int kk = 0; kk < DH / 4; ++kk) {
                const int a_off = (16 * qt + li) * SQ + 4 * kk + lq;
                s = __builtin_amdgcn_mfma_f32_16x16x4f32(Qs[a_off], kr[kk], s, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_16x16x4f32(dOs[a_off], vr[kk], dp, 0, 0, 0);
            }
            // s[r] = S[q = 16qt + 4lq + r][key = k0 + li]
            float p[4], ds[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = 16 * qt + 4 * lq + r;
                p[r] = kfl > 0.f ? expf(s[r] * scale - ls[q]) : 0.f;
                ds[r] = p[r] * (dp[r] - Dv[q]);
                dSs[q * SS + k0 + li] = ds[r] * scale;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qrow = (16 * qt + 4 * lq + r);
#pragma unroll
                for (int dt = 0; dt < DH / 16; ++dt) {
                    dv[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], dOs[qrow * SQ + 16 * dt + li], dv[dt], 0, 0, 0);
                    dk[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ds[r], Qs[qrow * SQ + 16 * dt + li], dk[dt], 0, 0, 0);
                }
            }
        }
        // dv[dt][r] = dV[k0 + 4lq + r][16dt + li]
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = k0 + 4 * lq + r;
            if (key < L) {
                gfloat* g = gb + (long)key * 3 * D + li;
#pragma unroll
                for (int dt = 0; dt < DH / 16; ++dt) {
                    g[D + 16 * dt] = dk[dt][r] * scale;
                    g[2 * D + 16 * dt] = dv[dt][r];
                }
            }
        }
    }
    __syncthreads();

    // ---- pass B: query stripes, dQ = (dS*scale) K
    for (int qt = wave; qt < NT; qt += 8) {
        floatx4 dq[DH / 16];
#pragma unroll
        for (int dt = 0; dt < DH / 16; ++dt) dq[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int kk = 0; kk < NT * 4; ++kk) {
            const float a = dSs[(16 * qt + li) * SS + 4 * kk + lq];
            const float* kr = &Ks[(4 * kk + lq) * SKB + li];
#pragma unroll
            for (int dt = 0; dt < DH / 16; ++dt)
                dq[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, kr[16 * dt], dq[dt], 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int q = 16 * qt + 4 * lq + r;
            if (q < L) {
                gfloat* g = gb + (long)q * 3 * D + li;
#pragma unroll
                for (int dt = 0; dt < DH / 16; ++dt) g[16 * dt] = dq[dt][r];
            }
        }
    }
}

size_t bwd_mfma_lds_bytes(int LP, int DH) {
    return sizeof(float) * ((size_t)LP * (DH + 4) * 2 + (size_t)LP * (DH + 16) + (size_t)LP * (LP + 4) + 3 * (size_t)LP);
}

template <int DH, int NT>
int launch_fwd_mfma(const float* qkv, const float* keep, float* ctx, float* lse, int N, int L, int H,
                    hipStream_t s) {
    hipLaunchKernelGGL((attn_fwd_mfma_kernel<DH, NT>), dim3(N * H), dim3(512), 0, s, qkv, keep, ctx, lse,
                       L, H, 1.0f / sqrtf((float)DH));
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

template <int DH, int NT>
int launch_bwd_mfma(const float* qkv, const float* keep, const float* ctx, const float* lse,
                    const float* dctx, float* dqkv, int N, int L, int H, hipStream_t s) {
    const size_t lds = bwd_mfma_lds_bytes(NT * 16, DH);
    PT_HIP(hipFuncSetAttribute((const void*)attn_bwd_mfma_kernel<DH, NT>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((attn_bwd_mfma_kernel<DH, NT>), dim3(N * H), dim3(512), lds, s, qkv, keep, ctx, lse,
                       dctx, dqkv, L, H, 1.0f / sqrtf((float)DH));
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

size_t fwd_lds_bytes(int L, int DH, int KPL) {
    return sizeof(float) * ((size_t)L * (DH + 1) * 2 + (size_t)L * DH + 4 * 64 * KPL + L);
}
size_t bwd_lds_bytes(int L, int DH) {
    return sizeof(float) * ((size_t)L * (DH + 1) * 4 + (size_t)L * (L + 1) + 3 * (size_t)L);
}

template <int DH, int KPL>
int launch_fwd(const float* qkv, const float* keep, float* ctx, float* lse, int N, int L, int H,
               hipStream_t s) {
    size_t lds = fwd_lds_bytes(L, DH, KPL);
    PT_HIP(hipFuncSetAttribute((const void*)attn_fwd_kernel<DH, KPL>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((attn_fwd_kernel<DH, KPL>), dim3(N * H), dim3(256), lds, s, qkv, keep, ctx,
                       lse, L, H, 1.0f / sqrtf((float)DH));
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

template <int DH, int KPL>
int launch_bwd(const float* qkv, const float* keep, const float* ctx, const float* lse,
               const float* dctx, float* dqkv, int N, int L, int H, hipStream_t s) {
    size_t lds = bwd_lds_bytes(L, DH);
    PT_HIP(hipFuncSetAttribute((const void*)attn_bwd_kernel<DH, KPL>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((attn_bwd_kernel<DH, KPL>), dim3(N * H), dim3(256), lds, s, qkv, keep, ctx,
                       lse, dctx, dqkv, L, H, 1.0f / sqrtf((float)DH));
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

}  // namespace

// LDS budget of one CDNA4 workgroup
static const size_t PT_LDS_MAX = 160 * 1024;

int pt_attn_supported(int L, int DH) {
    if (!(DH == 32 || DH == 64) || L > 256 || L < 1) return 0;
    return bwd_lds_bytes(L, DH) <= PT_LDS_MAX ? 1 : 0;
}

// MFMA kernels cover Lp = 16*ceil(L/16) <= 112 (Dh 64) / 128 (Dh 32) — the
// backward keeps Q, dO, K and dS for one (sample, head) in LDS; longer rows
// use the VALU kernels above (full-row softmax, LDS-resident P).
static const size_t PT_LDS_MFMA = 160 * 1024;
static int mfma_tiles(int L, int DH) {
    const int nt = pt_cdiv(L, 16);
    if (!(DH == 32 || DH == 64) || nt > 8) return 0;
    return bwd_mfma_lds_bytes(nt * 16, DH) <= PT_LDS_MFMA ? nt : 0;
}

#define PT_NT_SWITCH(DH, NT, CALL, ...)                                              \
    switch (NT) {                                                                    \
        case 1: return CALL<DH, 1>(__VA_ARGS__); case 2: return CALL<DH, 2>(__VA_ARGS__); \
        case 3: return CALL<DH, 3>(__VA_ARGS__); case 4: return CALL<DH, 4>(__VA_ARGS__); \
        case 5: return CALL<DH, 5>(__VA_ARGS__); case 6: return CALL<DH, 6>(__VA_ARGS__); \
        case 7: return CALL<DH, 7>(__VA_ARGS__); default: return CALL<DH, 8>(__VA_ARGS__); \
    }

int pt_attn_fwd(const float* qkv, const float* keep, float* ctx, float* lse, int N, int L, int H,
                int DH, hipStream_t s) {
    PT_REQUIRE(pt_attn_supported(L, DH), "attention: L=%d Dh=%d exceeds the fused kernel's LDS budget", L, DH);
    const int nt = mfma_tiles(L, DH);
    if (nt) {
        if (DH == 64) { PT_NT_SWITCH(64, nt, launch_fwd_mfma, qkv, keep, ctx, lse, N, L, H, s) }
        PT_NT_SWITCH(32, nt, launch_fwd_mfma, qkv, keep, ctx, lse, N, L, H, s)
    }
    const int kpl = pt_cdiv(L, 64);
    if (DH == 64) {
        if (kpl == 1) return launch_fwd<64, 1>(qkv, keep, ctx, lse, N, L, H, s);
        if (kpl == 2) return launch_fwd<64, 2>(qkv, keep, ctx, lse, N, L, H, s);
        return launch_fwd<64, 4>(qkv, keep, ctx, lse, N, L, H, s);
    }
    if (kpl == 1) return launch_fwd<32, 1>(qkv, keep, ctx, lse, N, L, H, s);
    if (kpl == 2) return launch_fwd<32, 2>(qkv, keep, ctx, lse, N, L, H, s);
    return launch_fwd<32, 4>(qkv, keep, ctx, lse, N, L, H, s);
}

int pt_attn_bwd(const float* qkv, const float* keep, const float* ctx, const float* lse,
                const float* dctx, float* dqkv, int N, int L, int H, int DH, hipStream_t s) {
    PT_REQUIRE(pt_attn_supported(L, DH), "attention bwd: L=%d Dh=%d exceeds the fused kernel's LDS budget", L, DH);
    const int nt = mfma_tiles(L, DH);
    if (nt) {
        if (DH == 64) { PT_NT_SWITCH(64, nt, launch_bwd_mfma, qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s) }
        PT_NT_SWITCH(32, nt, launch_bwd_mfma, qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s)
    }
    const int kpl = pt_cdiv(L, 64);
    if (DH == 64) {
        if (kpl == 1) return launch_bwd<64, 1>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s);
        if (kpl == 2) return launch_bwd<64, 2>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s);
        return launch_bwd<64, 4>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s);
    }
    if (kpl == 1) return launch_bwd<32, 1>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s);
    if (kpl == 2) return launch_bwd<32, 2>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s);
    return launch_bwd<32, 4>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s);
}
