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

int pt_attn_fwd(const float* qkv, const float* keep, float* ctx, float* lse, int N, int L, int H,
                int DH, hipStream_t s) {
    PT_REQUIRE(pt_attn_supported(L, DH), "attention: L=%d Dh=%d exceeds the fused kernel's LDS budget", L, DH);
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
