// Masked multi-head self-attention over padded entity tokens, fused per
// (sample, head); fp32, or bf16 products with fp32 softmax and accumulation.
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

#include <type_traits>

namespace {

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
// SIMD to overlap LDS reads with MFMAs.  In the forward and the stored-dS
// backward, products over the head dimension give lane group lq the dims
// 16kq + 4lq + e (e = 0..3) of both operands, and products with an output
// over the head dimension give lane li the output columns W li .. W li + W - 1
// (W = Dh / 16, one accumulator each): both are permutations applied to both
// operands alike, so every operand fragment is a row segment read as one
// vector and every output row segment is one vector store.

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// Four fp32 k-steps of one 16x16 product, lane (li, lq) supplying a[e] and
// b[e] for logical k = 4e + lq of the 16-k group: four
// v_mfma_f32_16x16x4_f32, or (BF, bf16 products with fp32 accumulation) one
// v_mfma_f32_16x16x16_bf16 on the same operands rounded to bf16 (RNE).  Its
// lane group lq, element e is k = 4 lq + e in the hardware's order — the
// same four k per lane, and A and B use the same map, so both forms sum the
// same products.
template <bool BF>
__device__ __forceinline__ floatx4 mfma4(const float (&a)[4], const float (&b)[4], floatx4 c) {
    if constexpr (BF) {
        const bf16x4 ah = {(__bf16)a[0], (__bf16)a[1], (__bf16)a[2], (__bf16)a[3]};
        const bf16x4 bh = {(__bf16)b[0], (__bf16)b[1], (__bf16)b[2], (__bf16)b[3]};
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bh, c, 0, 0, 0);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], c, 0, 0, 0);
        return c;
    }
}

// Element type T of qkv, ctx, dctx and dqkv: float, or __bf16 (the
// mixed-precision variant's activations, read and written in bf16; the
// products round their operands to bf16 anyway, so only the stored outputs
// and rowsum(dO o O) see the narrower type).
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 ld4(const __bf16* p) {
    const bf16x4 b = *reinterpret_cast<const bf16x4*>(p);
    return make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
}
__device__ __forceinline__ float tof(float v) { return v; }
__device__ __forceinline__ float tof(__bf16 v) { return (float)v; }
// LDS operand stores: fp32, or (bf16 products) bf16 — every LDS operand of
// the bf16 kernels feeds an MFMA that rounds it to bf16 anyway, so storing
// it rounded gives the same products with half the LDS
__device__ __forceinline__ void st_lds4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ void st_lds4(__bf16* p, float4 v) {
    *reinterpret_cast<bf16x4*>(p) = bf16x4{(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
}
// W (= Dh / 16) consecutive elements of a row as one 128- / 64-bit (bf16:
// 64- / 32-bit) access, in LDS or global memory
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <int W> __device__ __forceinline__ void ldw(const float* p, float (&o)[W]) {
    if constexpr (W == 4) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else {
        static_assert(W == 2, "W is Dh / 16: 2 or 4");
        const float2 v = *reinterpret_cast<const float2*>(p);
        o[0] = v.x; o[1] = v.y;
    }
}
template <int W> __device__ __forceinline__ void ldw(const __bf16* p, float (&o)[W]) {
    if constexpr (W == 4) {
        const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (float)v[i];
    } else {
        const bf16x2 v = *reinterpret_cast<const bf16x2*>(p);
        o[0] = (float)v[0]; o[1] = (float)v[1];
    }
}
template <int W> __device__ __forceinline__ void stw(float* p, const float (&v)[W]) {
    if constexpr (W == 4) *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    else *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
}
template <int W> __device__ __forceinline__ void stw(__bf16* p, const float (&v)[W]) {
    if constexpr (W == 4) *reinterpret_cast<bf16x4*>(p) = bf16x4{(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
    else *reinterpret_cast<bf16x2*>(p) = bf16x2{(__bf16)v[0], (__bf16)v[1]};
}

template <int DH, int NT, bool BF, typename T>   // NT = Lp / 16 key (and query) tiles
__global__ __launch_bounds__(512) void attn_fwd_mfma_kernel(const T* __restrict__ qkv,
        const float* __restrict__ keep, T* __restrict__ ctx, float* __restrict__ lse,
        int Lfix, int H, float scale, const int* __restrict__ coff) {
    constexpr int LP = NT * 16, SK = DH + 4, W = DH / 16;
    typedef typename std::conditional<BF, __bf16, float>::type LT;   // LDS operand type
    extern __shared__ float sm[];
    LT* Ks = reinterpret_cast<LT*>(sm);   // [LP][SK]
    LT* Vs = Ks + LP * SK;                // [LP][SK]
    float* kf = reinterpret_cast<float*>(Vs + LP * SK);   // [LP]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int n = blockIdx.x / H, h = blockIdx.x % H;
    // rows of sample n: [rb, rb + L) (compact layout) or [n*Lfix, (n+1)*Lfix)
    const long rb = coff ? (long)coff[n] : (long)n * Lfix;
    const int L = coff ? coff[n + 1] - coff[n] : Lfix;
    const int D = H * DH;
    // this sample's tiles (compact rows vary in length; the template covers the longest)
    const int ntl = min(NT, (L + 15) / 16);
    const T* base = qkv + rb * 3 * D + h * DH;
    // Q^T as the B operand: lane (li = query, lq) holds Q[q0+li][16kq+4lq+e]
    // at qb[4kq+e] (head dims 4lq..4lq+3 of each 16-group: one vector load);
    // the wave's first stripe is loaded before the K / V staging, so its
    // latency overlaps the staging's
    float qb[DH / 4];
    auto load_q = [&](int q0) {
        const bool qv = q0 + li < L;
#pragma unroll
        for (int kq = 0; kq < DH / 16; ++kq) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (qv) v = ld4(base + (long)(q0 + li) * 3 * D + 16 * kq + 4 * lq);
            qb[4 * kq] = v.x; qb[4 * kq + 1] = v.y; qb[4 * kq + 2] = v.z; qb[4 * kq + 3] = v.w;
        }
    };
    if (wave < ntl) load_q(wave * 16);
    // K / V staging in groups of SG row segments per thread: a group's loads
    // are all issued before its LDS stores, so the staging waits on memory
    // once per group instead of once per segment
    constexpr int SG = 4;
    const int nidx = ntl * 16 * (DH / 4);
    for (int i0 = tid; i0 < nidx; i0 += SG * 512) {
        float4 k4[SG], v4[SG];
#pragma unroll
        for (int u = 0; u < SG; ++u) {
            const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
            k4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            v4[u] = k4[u];
            if (idx < nidx && l < L) {
                const T* r = base + (long)l * 3 * D + c4;
                k4[u] = ld4(r + D);
                v4[u] = ld4(r + 2 * D);
            }
        }
#pragma unroll
        for (int u = 0; u < SG; ++u) {
            const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
            if (idx < nidx) {
                st_lds4(&Ks[l * SK + c4], k4[u]);
                st_lds4(&Vs[l * SK + c4], v4[u]);
            }
        }
    }
    for (int l = tid; l < LP; l += 512) kf[l] = l < L ? (keep[rb + l] != 0.f ? 1.f : 0.f) : -1.f;
    __syncthreads();

    for (int st = wave; st < ntl; st += 8) {
        const int q0 = st * 16;
        if (st != wave) load_q(q0);
        const bool qv = q0 + li < L;
        floatx4 o[DH / 16];
#pragma unroll
        for (int dt = 0; dt < DH / 16; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        // keys in chunks of up to CH tiles with a running max / sum (one
        // chunk when Lp <= 128, so the scores of a row stay in registers)
        constexpr int CH = NT < 8 ? NT : 8;
        float mx = -INFINITY, sum = 0.f;
#pragma unroll 1
        for (int c0 = 0; c0 < ntl; c0 += CH) {
            floatx4 sc[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                sc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
                if (c0 + j < ntl) {
#pragma unroll
                    for (int kq = 0; kq < DH / 16; ++kq) {
                        float a[4], b[4];
                        ldw<4>(Ks + (16 * (c0 + j) + li) * SK + 16 * kq + 4 * lq, a);
#pragma unroll
                        for (int e = 0; e < 4; ++e) b[e] = qb[4 * kq + e];
                        sc[j] = mfma4<BF>(a, b, sc[j]);
                    }
                }
            }
            // sc[j][r] = S^T[key = 16(c0+j) + 4lq + r][query = q0 + li]
            float cm = -INFINITY;
#pragma unroll
            for (int j = 0; j < CH; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float f = c0 + j < ntl ? kf[16 * (c0 + j) + 4 * lq + r] : -1.f;
                    const float v = f > 0.f ? sc[j][r] * scale : (f == 0.f ? -1e30f : -INFINITY);
                    sc[j][r] = v;
                    cm = fmaxf(cm, v);
                }
            cm = fmaxf(cm, __shfl_xor(cm, 16, 64));
            cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
            const float nm = fmaxf(mx, cm);
            const float alpha = expf(mx - nm);     // 0 on the first chunk
            float cs = 0.f;
#pragma unroll
            for (int j = 0; j < CH; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = expf(sc[j][r] - nm);
                    sc[j][r] = e;
                    cs += e;
                }
            cs += __shfl_xor(cs, 16, 64);
            cs += __shfl_xor(cs, 32, 64);
            sum = sum * alpha + cs;
            mx = nm;
            if (c0 > 0) {
                // rows of o are queries 4lq + r: take their factor from lane 4lq + r
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a = __shfl(alpha, 4 * lq + r, 64);
#pragma unroll
                    for (int dt = 0; dt < DH / 16; ++dt) o[dt][r] *= a;
                }
            }
            // O += P V over the permuted key order; output column W li + dt
            // of o[dt] (W = Dh / 16), so a lane's V operands of one key are W
            // consecutive columns (one vector LDS read)
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                if (c0 + j < ntl) {
                    const float a[4] = {sc[j][0], sc[j][1], sc[j][2], sc[j][3]};
                    float vv[4][W];
#pragma unroll
                    for (int r = 0; r < 4; ++r) ldw<W>(Vs + (16 * (c0 + j) + 4 * lq + r) * SK + W * li, vv[r]);
#pragma unroll
                    for (int dt = 0; dt < W; ++dt) {
                        const float b[4] = {vv[0][dt], vv[1][dt], vv[2][dt], vv[3][dt]};
                        o[dt] = mfma4<BF>(a, b, o[dt]);
                    }
                }
            }
        }
        // o[dt][r] = O[q0 + 4lq + r][W li + dt] * sum(query); normalise
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float inv = 1.0f / __shfl(sum, 4 * lq + r, 64);
            const int q = q0 + 4 * lq + r;
            if (q < L) {
                float v[W];
#pragma unroll
                for (int dt = 0; dt < W; ++dt) v[dt] = o[dt][r] * inv;
                stw<W>(ctx + (rb + q) * D + h * DH + W * li, v);
            }
        }
        if (lq == 0 && qv) lse[((long)n * H + h) * Lfix + q0 + li] = mx + logf(sum);
    }
}

// Backward.  Pass A walks key stripes: per query tile it recomputes
// S = Q K^T and dP = dO V^T with keys on lanes, forms P and
// dS = P (dP - rowsum(dO o O)), accumulates dV += P^T dO and dK += dS^T Q
// (register-r trick again, now over queries), and parks dS*scale.
// Pass B walks query stripes: dQ = dS K.
// GDS = false: dS is parked in LDS beside Q, dO and K (one workgroup per CU
// at Lp = 112, Dh 64).  GDS = true: dS goes to this workgroup's own slice of
// a global scratch (dsg + blockIdx * Lp * Lp, row-major, L2-resident between
// the passes: the writes and reads of one workgroup run on one CU, ordered
// by the barrier), and K is staged after pass A into the space Q and dO
// leave free, so the workgroup holds only Q and dO in LDS (two workgroups
// per CU: one's staging overlaps the other's products).  Pass B then reads
// dS rows as 128-bit loads, taking key 16 kq + 4 lq + e for lane group lq,
// element e (the K operand uses the same key order, SKB = Dh + 4 keeps those
// LDS reads conflict-free).
template <int DH, int NT, bool BF, typename T, bool GDS = false>
__global__ __launch_bounds__(512) void attn_bwd_mfma_kernel(const T* __restrict__ qkv,
        const float* __restrict__ keep, const T* __restrict__ ctx,
        const float* __restrict__ lse, const T* __restrict__ dctx,
        T* __restrict__ dqkv, int Lfix, int H, float scale, const int* __restrict__ coff,
        typename std::conditional<BF, __bf16, float>::type* __restrict__ dsg = nullptr) {
    constexpr int LP = NT * 16, SQ = DH + 4, SKB = GDS ? DH + 4 : DH + 16, SS = GDS ? LP : LP + 4, W = DH / 16;
    typedef typename std::conditional<BF, __bf16, float>::type LT;   // LDS operand type
    extern __shared__ float sm[];
    LT* Qs = reinterpret_cast<LT*>(sm);   // [LP][SQ]
    LT* dOs = Qs + LP * SQ;               // [LP][SQ]
    // K [LP][SKB]: after Q and dO (GDS: in Q's space once pass A is done)
    LT* Ks = GDS ? Qs : dOs + LP * SQ;
    // dS [LP][SS] (query-major): in LDS after K, or this workgroup's global slice
    LT* dSs = GDS ? dsg + (size_t)blockIdx.x * (LP * LP) : Ks + LP * SKB;
    float* ls = reinterpret_cast<float*>(GDS ? dOs + LP * SQ : Ks + LP * SKB + LP * SS);   // [LP]
    float* Dv = ls + LP;            // [LP]
    float* kf = Dv + LP;            // [LP]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int n = blockIdx.x / H, h = blockIdx.x % H;
    // rows of sample n: [rb, rb + L) (compact layout) or [n*Lfix, (n+1)*Lfix)
    const long rb = coff ? (long)coff[n] : (long)n * Lfix;
    const int L = coff ? coff[n + 1] - coff[n] : Lfix;
    const int D = H * DH;
    // this sample's tiles (compact rows vary in length; the template covers the longest)
    const int ntl = min(NT, (L + 15) / 16);
    const T* base = qkv + rb * 3 * D + h * DH;
    const T* ob = ctx + rb * D + h * DH;
    const T* dob = dctx + rb * D + h * DH;
    T* gb = dqkv + rb * 3 * D + h * DH;
    // pass A's B operands, loaded before the staging so their latency overlaps
    // it: lane (li = key, lq) holds K/V[k0+li][16kq+4lq+e] at [4kq+e] (the
    // head-dim order of the Q / dO operands below: one vector load each).
    // Wave w owns key stripe w (at most 8 stripes).
    static_assert(NT <= 8, "one key stripe per wave");
    const int kb = wave, k0 = kb * 16;
    const bool kv = k0 + li < L;
    float kr[DH / 4], vr[DH / 4];
#pragma unroll
    for (int kq = 0; kq < DH / 16; ++kq) {
        float4 k4 = make_float4(0.f, 0.f, 0.f, 0.f), v4 = k4;
        if (kb < ntl && kv) {
            k4 = ld4(base + (long)(k0 + li) * 3 * D + D + 16 * kq + 4 * lq);
            v4 = ld4(base + (long)(k0 + li) * 3 * D + 2 * D + 16 * kq + 4 * lq);
        }
        kr[4 * kq] = k4.x; kr[4 * kq + 1] = k4.y; kr[4 * kq + 2] = k4.z; kr[4 * kq + 3] = k4.w;
        vr[4 * kq] = v4.x; vr[4 * kq + 1] = v4.y; vr[4 * kq + 2] = v4.z; vr[4 * kq + 3] = v4.w;
    }
    // stage Q, dO, K and form Dv[q] = sum_d dO[q][d] O[q][d]: the DH/4 lanes
    // holding a row's 4-column partials are adjacent (512 is a multiple of
    // DH/4), so a butterfly over them gives the row sum (padded rows 0).
    // Segments go in groups of SG per thread, a group's loads all issued
    // before its stores (one wait on memory per group)
    constexpr int SG = GDS ? 4 : 2;
    const int nidx = ntl * 16 * (DH / 4);
    for (int i0 = tid; i0 < nidx; i0 += SG * 512) {
        float4 q4[SG], k4[SG], d4[SG], o4[SG];
#pragma unroll
        for (int u = 0; u < SG; ++u) {
            const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
            q4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            k4[u] = q4[u]; d4[u] = q4[u]; o4[u] = q4[u];
            if (idx < nidx && l < L) {
                const T* r = base + (long)l * 3 * D + c4;
                q4[u] = ld4(r);
                if (!GDS) k4[u] = ld4(r + D);
                d4[u] = ld4(dob + (long)l * D + c4);
                o4[u] = ld4(ob + (long)l * D + c4);
            }
        }
#pragma unroll
        for (int u = 0; u < SG; ++u) {
            const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
            if (idx < nidx) {
                st_lds4(&Qs[l * SQ + c4], q4[u]);
                st_lds4(&dOs[l * SQ + c4], d4[u]);
                if (!GDS) st_lds4(&Ks[l * SKB + c4], k4[u]);
                float part = ((d4[u].x * o4[u].x + d4[u].y * o4[u].y) + d4[u].z * o4[u].z) + d4[u].w * o4[u].w;
#pragma unroll
                for (int o = 1; o < DH / 4; o <<= 1) part += __shfl_xor(part, o, 64);
                if (c4 == 0) Dv[l] = part;
            }
        }
    }
    for (int l = tid; l < LP; l += 512) {
        kf[l] = l < L ? (keep[rb + l] != 0.f ? 1.f : 0.f) : 0.f;
        ls[l] = l < L ? lse[((long)n * H + h) * Lfix + l] : INFINITY;
    }
    __syncthreads();

    // ---- pass A: key stripes (wave kb's)
    if (kb < ntl) {
        const float kfl = kf[k0 + li];
        floatx4 dv[DH / 16], dk[DH / 16];
#pragma unroll
        for (int dt = 0; dt < DH / 16; ++dt) {
            dv[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
            dk[dt] = dv[dt];
        }
        for (int qt = 0; qt < ntl; ++qt) {
            floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f}, dp = s;
#pragma unroll
            for (int kq = 0; kq < DH / 16; ++kq) {
                float qa[4], da[4], kb4[4], vb4[4];
                const int a_off = (16 * qt + li) * SQ + 16 * kq + 4 * lq;
                ldw<4>(Qs + a_off, qa);
                ldw<4>(dOs + a_off, da);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kb4[e] = kr[4 * kq + e];
                    vb4[e] = vr[4 * kq + e];
                }
                s = mfma4<BF>(qa, kb4, s);
                dp = mfma4<BF>(da, vb4, dp);
            }
            // s[r] = S[q = 16qt + 4lq + r][key = k0 + li]
            float p[4], ds[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = 16 * qt + 4 * lq + r;
                p[r] = kfl > 0.f ? expf(s[r] * scale - ls[q]) : 0.f;
                ds[r] = p[r] * (dp[r] - Dv[q]);
                dSs[q * SS + k0 + li] = (LT)(ds[r] * scale);
            }
            // dV / dK output column W li + dt of dv[dt] / dk[dt]: a lane's dO / Q
            // operands of one query row are W consecutive columns
            float ow[4][W], qw[4][W];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qrow = 16 * qt + 4 * lq + r;
                ldw<W>(dOs + qrow * SQ + W * li, ow[r]);
                ldw<W>(Qs + qrow * SQ + W * li, qw[r]);
            }
#pragma unroll
            for (int dt = 0; dt < W; ++dt) {
                const float ob[4] = {ow[0][dt], ow[1][dt], ow[2][dt], ow[3][dt]};
                const float qb4[4] = {qw[0][dt], qw[1][dt], qw[2][dt], qw[3][dt]};
                dv[dt] = mfma4<BF>(p, ob, dv[dt]);
                dk[dt] = mfma4<BF>(ds, qb4, dk[dt]);
            }
        }
        // dv[dt][r] = dV[k0 + 4lq + r][W li + dt]
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = k0 + 4 * lq + r;
            if (key < L) {
                T* g = gb + (long)key * 3 * D + W * li;
                float kw[W], vw[W];
#pragma unroll
                for (int dt = 0; dt < W; ++dt) {
                    kw[dt] = dk[dt][r] * scale;
                    vw[dt] = dv[dt][r];
                }
                stw<W>(g + D, kw);
                stw<W>(g + 2 * D, vw);
            }
        }
    }
    __syncthreads();
    if (GDS) {
        // Q and dO are consumed: stage K into their space (its rows were just
        // read by pass A, so they come from L2), four segments' loads per
        // thread issued before their stores
        for (int i0 = tid; i0 < nidx; i0 += 4 * 512) {
            float4 k4[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
                k4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (idx < nidx && l < L) k4[u] = ld4(base + (long)l * 3 * D + D + c4);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
                if (idx < nidx) st_lds4(&Ks[l * SKB + c4], k4[u]);
            }
        }
        __syncthreads();
    }

    // ---- pass B: query stripes, dQ = (dS*scale) K
    for (int qt = wave; qt < ntl; qt += 8) {
        floatx4 dq[DH / 16];
#pragma unroll
        for (int dt = 0; dt < DH / 16; ++dt) dq[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        // GDS: the stripe's dS row segments (keys 16 kq + 4 lq + e: one 128-bit,
        // bf16 64-bit, load per key tile), all issued before the products
        float4 dsr[NT];
        if constexpr (GDS) {
#pragma unroll
            for (int kq = 0; kq < NT; ++kq)
                dsr[kq] = kq < ntl ? ld4(dSs + (16 * qt + li) * SS + 16 * kq + 4 * lq)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int kq = 0; kq < NT; ++kq) {
            if (kq >= ntl) break;
            float a[4];
            if constexpr (GDS) {
                a[0] = dsr[kq].x; a[1] = dsr[kq].y; a[2] = dsr[kq].z; a[3] = dsr[kq].w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) a[e] = (float)dSs[(16 * qt + li) * SS + 4 * (4 * kq + e) + lq];
            }
            // dQ output column W li + dt of dq[dt]: a lane's K operands of one
            // key are W consecutive columns
            float kw[4][W];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int key = GDS ? 16 * kq + 4 * lq + e : 4 * (4 * kq + e) + lq;
                ldw<W>(Ks + key * SKB + W * li, kw[e]);
            }
#pragma unroll
            for (int dt = 0; dt < W; ++dt) {
                const float b[4] = {kw[0][dt], kw[1][dt], kw[2][dt], kw[3][dt]};
                dq[dt] = mfma4<BF>(a, b, dq[dt]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int q = 16 * qt + 4 * lq + r;
            if (q < L) {
                float qv[W];
#pragma unroll
                for (int dt = 0; dt < W; ++dt) qv[dt] = dq[dt][r];
                stw<W>(gb + (long)q * 3 * D + W * li, qv);
            }
        }
    }
}

// Backward for rows too long to park dS (L x L) in LDS (the reference's
// 161-token trunk and 218-token critic at Dh 32), in two launches so two
// workgroups fit a CU (each stages two L x Dh operands, <= 80 KB):
// attn_bwd_kv_kernel stages Q and dO and runs pass A (per key stripe: S, dP
// recomputed, P, dS; dV += P^T dO, dK += dS^T Q) as above without parking
// dS; attn_bwd_q_kernel stages K and V and recomputes per query stripe S^T
// = K Q^T and dP^T = V dO^T (queries on lanes), then dQ += dS K with the
// register-r key permutation; its stripe's Q, dO and O rows are read
// straight into registers and rowsum(dO o O) is a butterfly over the four
// lanes holding a row.  Costs one more S and dP evaluation than the stored
// variant; both walk only the sample's own tiles.  Measured against one
// fused kernel holding Q, dO, K and V (four operands, one workgroup per
// CU): 623 vs 809 us at 512 x 161 rows x 8 heads, 973 vs 1266 us at 218
// rows; at 97 rows x Dh 64 the stored variant stays faster (286 vs 335 us).
template <int DH, int NT, bool BF, typename T>
__global__ __launch_bounds__(512) void attn_bwd_kv_kernel(const T* __restrict__ qkv,
        const float* __restrict__ keep, const T* __restrict__ ctx,
        const float* __restrict__ lse, const T* __restrict__ dctx,
        T* __restrict__ dqkv, int Lfix, int H, float scale, const int* __restrict__ coff) {
    constexpr int LP = NT * 16, SQ = DH + 4;
    extern __shared__ float sm[];
    float* Qs = sm;                 // [LP][SQ]
    float* dOs = Qs + LP * SQ;      // [LP][SQ]
    float* ls = dOs + LP * SQ;      // [LP]
    float* Dv = ls + LP;            // [LP]
    float* kf = Dv + LP;            // [LP]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int n = blockIdx.x / H, h = blockIdx.x % H;
    const long rb = coff ? (long)coff[n] : (long)n * Lfix;
    const int L = coff ? coff[n + 1] - coff[n] : Lfix;
    const int D = H * DH;
    const int ntl = min(NT, (L + 15) / 16);
    const T* base = qkv + rb * 3 * D + h * DH;
    const T* ob = ctx + rb * D + h * DH;
    const T* dob = dctx + rb * D + h * DH;
    T* gb = dqkv + rb * 3 * D + h * DH;
    // staging in groups of four row segments per thread, loads before stores
    const int nidx = ntl * 16 * (DH / 4);
    for (int i0 = tid; i0 < nidx; i0 += 4 * 512) {
        float4 q4[4], d4[4], o4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
            q4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            d4[u] = q4[u]; o4[u] = q4[u];
            if (idx < nidx && l < L) {
                q4[u] = ld4(base + (long)l * 3 * D + c4);
                d4[u] = ld4(dob + (long)l * D + c4);
                o4[u] = ld4(ob + (long)l * D + c4);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
            if (idx < nidx) {
                *reinterpret_cast<float4*>(&Qs[l * SQ + c4]) = q4[u];
                *reinterpret_cast<float4*>(&dOs[l * SQ + c4]) = d4[u];
                float part = ((d4[u].x * o4[u].x + d4[u].y * o4[u].y) + d4[u].z * o4[u].z) + d4[u].w * o4[u].w;
#pragma unroll
                for (int o = 1; o < DH / 4; o <<= 1) part += __shfl_xor(part, o, 64);
                if (c4 == 0) Dv[l] = part;
            }
        }
    }
    for (int l = tid; l < LP; l += 512) {
        kf[l] = l < L ? (keep[rb + l] != 0.f ? 1.f : 0.f) : 0.f;
        ls[l] = l < L ? lse[((long)n * H + h) * Lfix + l] : INFINITY;
    }
    __syncthreads();
    for (int kb = wave; kb < ntl; kb += 8) {
        const int k0 = kb * 16;
        const bool kv = k0 + li < L;
        float kr[DH / 4], vr[DH / 4];   // B operands: lane (li = key, lq) holds K/V[k0+li][4kk+lq]
#pragma unroll
        for (int kk = 0; kk < DH / 4; ++kk) {
            kr[kk] = kv ? tof(base[(long)(k0 + li) * 3 * D + D + 4 * kk + lq]) : 0.f;
            vr[kk] = kv ? tof(base[(long)(k0 + li) * 3 * D + 2 * D + 4 * kk + lq]) : 0.f;
        }
        const float kfl = kf[k0 + li];
        floatx4 dv[DH / 16], dk[DH / 16];
#pragma unroll
        for (int dt = 0; dt < DH / 16; ++dt) {
            dv[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
            dk[dt] = dv[dt];
        }
        for (int qt = 0; qt < ntl; ++qt) {
            floatx4 sc = floatx4{0.f, 0.f, 0.f, 0.f}, dp = sc;
#pragma unroll
            for (int kq = 0; kq < DH / 16; ++kq) {
                float qa[4], da[4], kb4[4], vb4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int a_off = (16 * qt + li) * SQ + 4 * (4 * kq + e) + lq;
                    qa[e] = Qs[a_off];
                    da[e] = dOs[a_off];
                    kb4[e] = kr[4 * kq + e];
                    vb4[e] = vr[4 * kq + e];
                }
                sc = mfma4<BF>(qa, kb4, sc);
                dp = mfma4<BF>(da, vb4, dp);
            }
            // sc[r] = S[q = 16qt + 4lq + r][key = k0 + li]
            float p[4], ds[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = 16 * qt + 4 * lq + r;
                p[r] = kfl > 0.f ? expf(sc[r] * scale - ls[q]) : 0.f;
                ds[r] = p[r] * (dp[r] - Dv[q]);
            }
#pragma unroll
            for (int dt = 0; dt < DH / 16; ++dt) {
                float obr[4], qb4[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int qrow = 16 * qt + 4 * lq + r;
                    obr[r] = dOs[qrow * SQ + 16 * dt + li];
                    qb4[r] = Qs[qrow * SQ + 16 * dt + li];
                }
                dv[dt] = mfma4<BF>(p, obr, dv[dt]);
                dk[dt] = mfma4<BF>(ds, qb4, dk[dt]);
            }
        }
        // dv[dt][r] = dV[k0 + 4lq + r][16dt + li]
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = k0 + 4 * lq + r;
            if (key < L) {
                T* g = gb + (long)key * 3 * D + li;
#pragma unroll
                for (int dt = 0; dt < DH / 16; ++dt) {
                    g[D + 16 * dt] = (T)(dk[dt][r] * scale);
                    g[2 * D + 16 * dt] = (T)dv[dt][r];
                }
            }
        }
    }
}

template <int DH, int NT, bool BF, typename T>
__global__ __launch_bounds__(512) void attn_bwd_q_kernel(const T* __restrict__ qkv,
        const float* __restrict__ keep, const T* __restrict__ ctx,
        const float* __restrict__ lse, const T* __restrict__ dctx,
        T* __restrict__ dqkv, int Lfix, int H, float scale, const int* __restrict__ coff) {
    constexpr int LP = NT * 16, SQ = DH + 4;
    extern __shared__ float sm[];
    float* Ks = sm;                 // [LP][SQ]
    float* Vs = Ks + LP * SQ;       // [LP][SQ]
    float* kf = Vs + LP * SQ;       // [LP]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int n = blockIdx.x / H, h = blockIdx.x % H;
    const long rb = coff ? (long)coff[n] : (long)n * Lfix;
    const int L = coff ? coff[n + 1] - coff[n] : Lfix;
    const int D = H * DH;
    const int ntl = min(NT, (L + 15) / 16);
    const T* base = qkv + rb * 3 * D + h * DH;
    const T* ob = ctx + rb * D + h * DH;
    const T* dob = dctx + rb * D + h * DH;
    T* gb = dqkv + rb * 3 * D + h * DH;
    // staging in groups of four row segments per thread, loads before stores
    const int nidx = ntl * 16 * (DH / 4);
    for (int i0 = tid; i0 < nidx; i0 += 4 * 512) {
        float4 k4[4], v4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
            k4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            v4[u] = k4[u];
            if (idx < nidx && l < L) {
                const T* r = base + (long)l * 3 * D + c4;
                k4[u] = ld4(r + D);
                v4[u] = ld4(r + 2 * D);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = i0 + u * 512, l = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
            if (idx < nidx) {
                *reinterpret_cast<float4*>(&Ks[l * SQ + c4]) = k4[u];
                *reinterpret_cast<float4*>(&Vs[l * SQ + c4]) = v4[u];
            }
        }
    }
    for (int l = tid; l < LP; l += 512) kf[l] = l < L ? (keep[rb + l] != 0.f ? 1.f : 0.f) : 0.f;
    __syncthreads();
    for (int qt = wave; qt < ntl; qt += 8) {
        const int q0 = qt * 16;
        const bool qv = q0 + li < L;
        float qb[DH / 4], db[DH / 4];   // B operands: lane (li = query, lq) holds Q/dO[q0+li][4kk+lq]
        float dvq = 0.f;
#pragma unroll
        for (int kk = 0; kk < DH / 4; ++kk) {
            const long qr = (long)(q0 + li);
            qb[kk] = qv ? tof(base[qr * 3 * D + 4 * kk + lq]) : 0.f;
            db[kk] = qv ? tof(dob[qr * D + 4 * kk + lq]) : 0.f;
            dvq += db[kk] * (qv ? tof(ob[qr * D + 4 * kk + lq]) : 0.f);
        }
        // rowsum(dO o O) of query q0 + li: its four lane groups
        dvq += __shfl_xor(dvq, 16, 64);
        dvq += __shfl_xor(dvq, 32, 64);
        const float lsq = qv ? lse[((long)n * H + h) * Lfix + q0 + li] : INFINITY;
        floatx4 dq[DH / 16];
#pragma unroll
        for (int dt = 0; dt < DH / 16; ++dt) dq[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int J = 0; J < ntl; ++J) {
            floatx4 st = floatx4{0.f, 0.f, 0.f, 0.f}, dpt = st;
#pragma unroll
            for (int kq = 0; kq < DH / 16; ++kq) {
                float ka[4], va[4], qb4[4], db4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int a_off = (16 * J + li) * SQ + 4 * (4 * kq + e) + lq;
                    ka[e] = Ks[a_off];
                    va[e] = Vs[a_off];
                    qb4[e] = qb[4 * kq + e];
                    db4[e] = db[4 * kq + e];
                }
                st = mfma4<BF>(ka, qb4, st);
                dpt = mfma4<BF>(va, db4, dpt);
            }
            // st[r] = S^T[key = 16J + 4lq + r][query = q0 + li]
            float dst[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = 16 * J + 4 * lq + r;
                const float pt = kf[key] > 0.f ? expf(st[r] * scale - lsq) : 0.f;
                dst[r] = pt * (dpt[r] - dvq) * scale;
            }
#pragma unroll
            for (int dt = 0; dt < DH / 16; ++dt) {
                float b[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) b[r] = Ks[(16 * J + 4 * lq + r) * SQ + li + 16 * dt];
                dq[dt] = mfma4<BF>(dst, b, dq[dt]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int q = q0 + 4 * lq + r;
            if (q < L) {
                T* g = gb + (long)q * 3 * D + li;
#pragma unroll
                for (int dt = 0; dt < DH / 16; ++dt) g[16 * dt] = (T)dq[dt][r];
            }
        }
    }
}

size_t bwd_split_lds_bytes(int LP, int DH) { return sizeof(float) * ((size_t)LP * (DH + 4) * 2 + 3 * (size_t)LP); }

template <int DH, int NT, bool BF, bool IO16>
int launch_bwd_split(const float* qkv, const float* keep, const float* ctx, const float* lse,
                     const float* dctx, float* dqkv, int N, int L, int H, hipStream_t s, const int* coff) {
    typedef typename std::conditional<IO16, __bf16, float>::type T;
    const size_t lds = bwd_split_lds_bytes(NT * 16, DH);
    PT_HIP(hipFuncSetAttribute((const void*)attn_bwd_kv_kernel<DH, NT, BF, T>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    PT_HIP(hipFuncSetAttribute((const void*)attn_bwd_q_kernel<DH, NT, BF, T>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const float sc = 1.0f / sqrtf((float)DH);
    hipLaunchKernelGGL((attn_bwd_kv_kernel<DH, NT, BF, T>), dim3(N * H), dim3(512), lds, s,
                       reinterpret_cast<const T*>(qkv), keep, reinterpret_cast<const T*>(ctx), lse,
                       reinterpret_cast<const T*>(dctx), reinterpret_cast<T*>(dqkv), L, H, sc, coff);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL((attn_bwd_q_kernel<DH, NT, BF, T>), dim3(N * H), dim3(512), lds, s,
                       reinterpret_cast<const T*>(qkv), keep, reinterpret_cast<const T*>(ctx), lse,
                       reinterpret_cast<const T*>(dctx), reinterpret_cast<T*>(dqkv), L, H, sc, coff);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

// es: bytes per LDS operand element (4, or 2 for the bf16-product kernels)
size_t fwd_mfma_lds_bytes(int LP, int DH, size_t es = 4) {
    return es * (size_t)LP * (DH + 4) * 2 + sizeof(float) * (size_t)LP;
}

size_t bwd_mfma_lds_bytes(int LP, int DH, size_t es = 4) {
    return es * ((size_t)LP * (DH + 4) * 2 + (size_t)LP * (DH + 16) + (size_t)LP * (LP + 4)) +
           sizeof(float) * 3 * (size_t)LP;
}

// BF: bf16 products; IO16 (with BF): qkv / ctx / dctx / dqkv stored in bf16
template <int DH, int NT, bool BF, bool IO16>
int launch_fwd_mfma(const float* qkv, const float* keep, float* ctx, float* lse, int N, int L, int H,
                    hipStream_t s, const int* coff) {
    typedef typename std::conditional<IO16, __bf16, float>::type T;
    const size_t lds = fwd_mfma_lds_bytes(NT * 16, DH, BF ? 2 : 4);
    PT_HIP(hipFuncSetAttribute((const void*)attn_fwd_mfma_kernel<DH, NT, BF, T>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((attn_fwd_mfma_kernel<DH, NT, BF, T>), dim3(N * H), dim3(512), lds, s,
                       reinterpret_cast<const T*>(qkv), keep, reinterpret_cast<T*>(ctx), lse, L, H,
                       1.0f / sqrtf((float)DH), coff);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

// dS in global scratch: LDS holds Q and dO (K later in Q's space)
size_t bwd_gds_lds_bytes(int LP, int DH, size_t es = 4) {
    return es * (size_t)LP * (DH + 4) * 2 + sizeof(float) * 3 * (size_t)LP;
}

// dsg: the global dS scratch (N * H * Lp * Lp operand elements) or null for
// the variant that parks dS in LDS
template <int DH, int NT, bool BF, bool IO16>
int launch_bwd_mfma(const float* qkv, const float* keep, const float* ctx, const float* lse,
                    const float* dctx, float* dqkv, int N, int L, int H, hipStream_t s, const int* coff,
                    void* dsg) {
    typedef typename std::conditional<IO16, __bf16, float>::type T;
    typedef typename std::conditional<BF, __bf16, float>::type LT;
    const float sc = 1.0f / sqrtf((float)DH);
    if (dsg) {
        const size_t lds = bwd_gds_lds_bytes(NT * 16, DH, BF ? 2 : 4);
        PT_HIP(hipFuncSetAttribute((const void*)attn_bwd_mfma_kernel<DH, NT, BF, T, true>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL((attn_bwd_mfma_kernel<DH, NT, BF, T, true>), dim3(N * H), dim3(512), lds, s,
                           reinterpret_cast<const T*>(qkv), keep, reinterpret_cast<const T*>(ctx), lse,
                           reinterpret_cast<const T*>(dctx), reinterpret_cast<T*>(dqkv), L, H, sc, coff,
                           reinterpret_cast<LT*>(dsg));
        PT_LAUNCH_CHECK();
        return PTCG_OK;
    }
    const size_t lds = bwd_mfma_lds_bytes(NT * 16, DH, BF ? 2 : 4);
    PT_HIP(hipFuncSetAttribute((const void*)attn_bwd_mfma_kernel<DH, NT, BF, T>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((attn_bwd_mfma_kernel<DH, NT, BF, T>), dim3(N * H), dim3(512), lds, s,
                       reinterpret_cast<const T*>(qkv), keep, reinterpret_cast<const T*>(ctx), lse,
                       reinterpret_cast<const T*>(dctx), reinterpret_cast<T*>(dqkv), L, H, sc, coff,
                       nullptr);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

}  // namespace

// LDS budget of one CDNA4 workgroup
static const size_t PT_LDS_MAX = 160 * 1024;

// Kernel choice per (L, Dh), Lp = 16 * ceil(L / 16) = 16 * nt, nt <= 16
// (L <= 256) at Dh 32 and 64: forward MFMA; backward MFMA with dS parked in
// LDS when it fits (nt <= 8), else the split recompute pair.  At Dh 64 the
// split pair stages up to 80 KB per workgroup through nt = 9 (two
// workgroups per CU) and up to 139 KB at nt = 16 (one per CU): the
// reference variant's 161-position trunk and 218-position critic with
// 4 heads of 64 (native/model/ptcg_model.cu:19-21 sizes the trunk by
// d_model / heads).
static const int PT_NT_MAX32 = 16, PT_NT_MAX64 = 16;
static int nt_max(int DH) { return DH == 32 ? PT_NT_MAX32 : (DH == 64 ? PT_NT_MAX64 : 0); }
static int fwd_tiles(int L, int DH) {
    const int nt = pt_cdiv(L, 16);
    return (nt <= nt_max(DH) && fwd_mfma_lds_bytes(nt * 16, DH) <= PT_LDS_MAX) ? nt : 0;
}
static int bwd_store_tiles(int L, int DH) {
    const int nt = pt_cdiv(L, 16);
    if (!(DH == 32 || DH == 64) || nt > 8) return 0;
    return bwd_mfma_lds_bytes(nt * 16, DH) <= PT_LDS_MAX ? nt : 0;
}
static int bwd_split_tiles(int L, int DH) {
    const int nt = pt_cdiv(L, 16);
    return (nt <= nt_max(DH) && bwd_split_lds_bytes(nt * 16, DH) <= PT_LDS_MAX) ? nt : 0;
}

int pt_attn_supported(int L, int DH) {
    if (!(DH == 32 || DH == 64) || L > 256 || L < 1) return 0;
    return (fwd_tiles(L, DH) && (bwd_store_tiles(L, DH) || bwd_split_tiles(L, DH))) ? 1 : 0;
}

// (used inside the BF / IO16-templated dispatchers below)
#define PT_NT_CASE(DH, N, CALL, ...) case N: return CALL<DH, N, BF, IO16>(__VA_ARGS__);
#define PT_NT_SWITCH8(DH, NT, CALL, ...)                                                              \
    switch (NT) {                                                                                     \
        PT_NT_CASE(DH, 1, CALL, __VA_ARGS__) PT_NT_CASE(DH, 2, CALL, __VA_ARGS__)                     \
        PT_NT_CASE(DH, 3, CALL, __VA_ARGS__) PT_NT_CASE(DH, 4, CALL, __VA_ARGS__)                     \
        PT_NT_CASE(DH, 5, CALL, __VA_ARGS__) PT_NT_CASE(DH, 6, CALL, __VA_ARGS__)                     \
        PT_NT_CASE(DH, 7, CALL, __VA_ARGS__) PT_NT_CASE(DH, 8, CALL, __VA_ARGS__)                     \
        default: break;                                                                               \
    }
#define PT_NT_SWITCH_HI(DH, NT, CALL, ...)                                                            \
    switch (NT) {                                                                                     \
        PT_NT_CASE(DH, 9, CALL, __VA_ARGS__) PT_NT_CASE(DH, 10, CALL, __VA_ARGS__)                    \
        PT_NT_CASE(DH, 11, CALL, __VA_ARGS__) PT_NT_CASE(DH, 12, CALL, __VA_ARGS__)                   \
        PT_NT_CASE(DH, 13, CALL, __VA_ARGS__) PT_NT_CASE(DH, 14, CALL, __VA_ARGS__)                   \
        PT_NT_CASE(DH, 15, CALL, __VA_ARGS__) PT_NT_CASE(DH, 16, CALL, __VA_ARGS__)                   \
        default: break;                                                                               \
    }

template <bool BF, bool IO16>
static int attn_fwd_dispatch(const float* qkv, const float* keep, float* ctx, float* lse, int N, int L, int H,
                             int DH, hipStream_t s, const int* coff) {
    const int nt = fwd_tiles(L, DH);
    if (nt && DH == 64) {
        PT_NT_SWITCH8(64, nt, launch_fwd_mfma, qkv, keep, ctx, lse, N, L, H, s, coff)
        PT_NT_SWITCH_HI(64, nt, launch_fwd_mfma, qkv, keep, ctx, lse, N, L, H, s, coff)
    } else if (nt) {
        PT_NT_SWITCH8(32, nt, launch_fwd_mfma, qkv, keep, ctx, lse, N, L, H, s, coff)
        PT_NT_SWITCH_HI(32, nt, launch_fwd_mfma, qkv, keep, ctx, lse, N, L, H, s, coff)
    }
    PT_REQUIRE(false, "attention: no kernel for L=%d Dh=%d", L, DH);
}

template <bool BF, bool IO16>
static int attn_bwd_dispatch(const float* qkv, const float* keep, const float* ctx, const float* lse,
                             const float* dctx, float* dqkv, int N, int L, int H, int DH, hipStream_t s,
                             const int* coff, void* dsg) {
    int nt = bwd_store_tiles(L, DH);
    if (nt) {
        if (DH == 64) { PT_NT_SWITCH8(64, nt, launch_bwd_mfma, qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s, coff, dsg) }
        else { PT_NT_SWITCH8(32, nt, launch_bwd_mfma, qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s, coff, dsg) }
    }
    nt = bwd_split_tiles(L, DH);
    if (nt && DH == 64) {
        PT_NT_SWITCH8(64, nt, launch_bwd_split, qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s, coff)
        PT_NT_SWITCH_HI(64, nt, launch_bwd_split, qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s, coff)
    } else if (nt) {
        PT_NT_SWITCH8(32, nt, launch_bwd_split, qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s, coff)
        PT_NT_SWITCH_HI(32, nt, launch_bwd_split, qkv, keep, ctx, lse, dctx, dqkv, N, L, H, s, coff)
    }
    PT_REQUIRE(false, "attention bwd: no kernel for L=%d Dh=%d", L, DH);
}

int pt_attn_fwd(const float* qkv, const float* keep, float* ctx, float* lse, int N, int L, int H,
                int DH, hipStream_t s, const int* coff, int prec) {
    PT_REQUIRE(pt_attn_supported(L, DH), "attention: L=%d Dh=%d exceeds the fused kernels' LDS budget", L, DH);
    if (prec == 2) return attn_fwd_dispatch<true, true>(qkv, keep, ctx, lse, N, L, H, DH, s, coff);
    return prec ? attn_fwd_dispatch<true, false>(qkv, keep, ctx, lse, N, L, H, DH, s, coff)
                : attn_fwd_dispatch<false, false>(qkv, keep, ctx, lse, N, L, H, DH, s, coff);
}

size_t pt_attn_bwd_ws_bytes(int N, int L, int H, int DH, int prec) {
    if (!pt_attn_supported(L, DH)) return 0;
    const int nt = bwd_store_tiles(L, DH);
    if (!nt) return 0;   // the split pair keeps nothing between its launches
    return (size_t)N * H * (size_t)(nt * 16) * (nt * 16) * (prec ? 2 : 4);
}

int pt_attn_bwd(const float* qkv, const float* keep, const float* ctx, const float* lse,
                const float* dctx, float* dqkv, int N, int L, int H, int DH, hipStream_t s, const int* coff,
                int prec, void* ws, size_t ws_bytes) {
    PT_REQUIRE(pt_attn_supported(L, DH), "attention bwd: L=%d Dh=%d exceeds the fused kernels' LDS budget", L, DH);
    const size_t need = pt_attn_bwd_ws_bytes(N, L, H, DH, prec);
    void* dsg = (ws != nullptr && need > 0 && ws_bytes >= need) ? ws : nullptr;
    if (prec == 2) return attn_bwd_dispatch<true, true>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, DH, s, coff, dsg);
    return prec ? attn_bwd_dispatch<true, false>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, DH, s, coff, dsg)
                : attn_bwd_dispatch<false, false>(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, DH, s, coff, dsg);
}

// Which kernels a shape takes (for tests): bit 0 forward, bit 1 backward
// with dS in LDS, bit 2 backward recompute; -1 unsupported.
int pt_attn_path(int L, int DH) {
    if (!pt_attn_supported(L, DH)) return -1;
    int f = fwd_tiles(L, DH) ? 1 : 0;
    if (bwd_store_tiles(L, DH)) f |= 2;
    else if (bwd_split_tiles(L, DH)) f |= 4;
    return f;
}
