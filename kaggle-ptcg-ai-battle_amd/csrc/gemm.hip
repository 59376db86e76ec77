// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x4_f32), LDS-staged.
//
// Replaces the reference's cuBLAS GemmEx wrappers pt_gemm / pt_linear /
// pt_linear_bwd / pt_bias_grad (native/model/ptcg_kernels.cuh:42-108) with
// one templated kernel: 128x128 block tile, BK = 16, 256 threads = 4 waves
// in a 2x2 grid, each wave a 64x64 sub-tile of 4x4 MFMA 16x16 tiles.
// Global->LDS moves 128-bit vectors along whichever dimension is contiguous
// in memory, double buffered (the prefetch of tile t+1 overlaps the MFMAs of
// tile t), and is stored without transposition; the MFMA k order is chosen
// so a k-contiguous fragment is a single 128-bit LDS read per four MFMA
// steps.  Tiles are ordered per XCD (L2 reuse of the A rows).  Epilogues
// fuse bias, exact GELU (keeping the pre-activation), residual add and the
// GELU backward multiply.  Weight gradients (K = rows, small M*N) split K
// across blocks and sum the partials in a fixed order, so results do not
// depend on scheduling (the reference accumulates with atomics).
#include "common.h"

#include <vector>

namespace {

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int NT = 256;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ bf16x4 to_bf16x4(float a, float b, float c, float d) {
    return bf16x4{(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
}
// LDS layouts.  A k-contiguous operand is staged [row][k] (stride BK+4: the
// 128-bit fragment reads of 8 consecutive rows cover all 32 banks); an
// m-contiguous operand is staged [k][row] (stride BM+4: rows 4 apart land 16
// banks apart).  Both use the same k order: lane group lq of an MFMA step kk
// supplies k = 4*lq + kk, so a [row][k] fragment is one 128-bit read serving
// four MFMA steps.
constexpr int SK = BK + 4;      // [row][k] stride
constexpr int SM = BM + 4;      // [k][row] stride
template <bool T> struct Stage { static constexpr int floats = T ? BK * SM : BM * SK; };

// XCD-aware tile order: workgroups are dealt round-robin to the 8 XCDs, so
// hand XCD x a contiguous range of logical tiles (all N-tiles of a run of
// M-tiles) and the A rows stay in that XCD's L2.
__device__ __forceinline__ void tile_of(int b, int tiles, int tn, int& tm_i, int& tn_i) {
    int lb = b;
    if ((tiles & 7) == 0) lb = (b & 7) * (tiles >> 3) + (b >> 3);
    tm_i = lb / tn;
    tn_i = lb % tn;
}
// effective shape of a launch: the device row / reduction counts when given
__device__ __forceinline__ GemmArgs gemm_shape(const GemmArgs& g0) {
    GemmArgs g = g0;
    if (g.Mdev) g.M = min(*g.Mdev, g.M);
    if (g.Kdev) g.K = min(*g.Kdev, g.K);
    return g;
}

// The launch's logical tile range [g.tile0, g.tile0 + count), count taken
// from the effective (device) row count: blocks are dealt round-robin to the
// 8 XCDs, so XCD x gets the contiguous logical range starting at
// x*q + min(x, r) (count = 8q + r) — every XCD gets work and keeps its A rows
// in its own L2.  Returns false for blocks beyond the count.
__device__ __forceinline__ bool tile_of_range(const GemmArgs& g, int tn, int& tm_i, int& tn_i, int b) {
    const int count = g.ntiles ? g.ntiles : ((g.M + BM - 1) / BM) * tn;
    if (b >= count) return false;
    const int q = count >> 3, r = count & 7, x = b & 7;
    const int lb = g.tile0 + x * q + min(x, r) + (b >> 3);
    tm_i = lb / tn;
    tn_i = lb % tn;
    return true;
}

// bf16 activations (OB): C and C2 hold bf16 (round to nearest even), and so
// does R for EPI_MUL (the GELU derivative the forward stored in bf16); the
// residual R of EPI_BIAS_RESID and the bias stay fp32
typedef __attribute__((address_space(1))) __bf16 gbf16;
typedef __attribute__((address_space(1))) bf16x4 gbf16x4;
__device__ __forceinline__ __bf16* bfp(float* p) { return reinterpret_cast<__bf16*>(p); }
__device__ __forceinline__ const __bf16* bfp(const float* p) { return reinterpret_cast<const __bf16*>(p); }
__device__ __forceinline__ void st_b1(float* base, long i, float v) { *(gbf16*)(bfp(base) + i) = (__bf16)v; }
__device__ __forceinline__ float ld_b1(const float* base, long i) { return (float)*(const gbf16*)(bfp(base) + i); }
__device__ __forceinline__ void st_b4(float* base, long i, floatx4 v) {
    *(gbf16x4*)(bfp(base) + i) = to_bf16x4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ floatx4 ld_b4(const float* base, long i) {
    const bf16x4 b = *(const gbf16x4*)(bfp(base) + i);
    return floatx4{(float)b[0], (float)b[1], (float)b[2], (float)b[3]};
}

template <int EPI>
__device__ __forceinline__ void epi_store_bf(const GemmArgs& g, int m, int n, float v) {
    const long c = (long)m * g.ldc + n;
    if (EPI == EPI_STORE) {
        st_b1(g.C, c, v);
    } else if (EPI == EPI_BIAS) {
        st_b1(g.C, c, v + g.bias[n]);
    } else if (EPI == EPI_BIAS_GELU_D) {
        float gv, gd;
        pt_gelu_both_bf(v + g.bias[n], gv, gd);
        st_b1(g.C, c, gd);
        st_b1(g.C2, (long)m * g.ldc2 + n, gv);
    } else if (EPI == EPI_MUL) {
        st_b1(g.C, c, v * ld_b1(g.R, (long)m * g.ldr + n));
    } else if (EPI == EPI_BIAS_RESID) {
        st_b1(g.C, c, v + g.bias[n] + g.R[(long)m * g.ldr + n]);
    }
}

// one output element through the epilogue
template <int EPI, bool OB = false>
__device__ __forceinline__ void epi_store(const GemmArgs& g, int m, int n, float v) {
    if (OB) {
        epi_store_bf<EPI>(g, m, n, v);
    } else if (EPI == EPI_STORE) {
        g.C[(long)m * g.ldc + n] = v;
    } else if (EPI == EPI_BIAS) {
        g.C[(long)m * g.ldc + n] = v + g.bias[n];
    } else if (EPI == EPI_BIAS_GELU) {
        v += g.bias[n];
        g.C[(long)m * g.ldc + n] = v;
        g.C2[(long)m * g.ldc2 + n] = pt_gelu(v);
    } else if (EPI == EPI_BIAS_RESID) {
        g.C[(long)m * g.ldc + n] = v + g.bias[n] + g.R[(long)m * g.ldr + n];
    } else if (EPI == EPI_GELU_BWD) {
        g.C[(long)m * g.ldc + n] = v * pt_gelu_grad(g.R[(long)m * g.ldr + n]);
    } else if (EPI == EPI_BIAS_GELU_D) {
        float gv, gd;
        pt_gelu_both(v + g.bias[n], gv, gd);
        g.C[(long)m * g.ldc + n] = gd;
        g.C2[(long)m * g.ldc2 + n] = gv;
    } else if (EPI == EPI_MUL) {
        g.C[(long)m * g.ldc + n] = v * g.R[(long)m * g.ldr + n];
    } else if (EPI == EPI_AXPBY) {
        g.C[(long)m * g.ldc + n] = g.alpha * v + g.beta * g.R[(long)m * g.ldr + n];
    } else if (EPI == EPI_ACCUM) {
        g.C[(long)m * g.ldc + n] += v;
    }
}

// four consecutive outputs C[m][n..n+3] through the epilogue (128-bit
// accesses: the caller checked alignment and n + 3 < N); same arithmetic
// order as epi_store
__device__ __forceinline__ void st_g4(float* p, floatx4 v) { *(gfloatx4*)(gfloat*)p = v; }
__device__ __forceinline__ floatx4 ld_v4(const float* p) { return *(const gfloatx4*)(const gfloat*)p; }

template <int EPI>
__device__ __forceinline__ void epi_store4_bf(const GemmArgs& g, int m, int n, floatx4 v) {
    const long c = (long)m * g.ldc + n;
    if (EPI == EPI_STORE) {
        st_b4(g.C, c, v);
    } else if (EPI == EPI_BIAS) {
        st_b4(g.C, c, v + ld_v4(g.bias + n));
    } else if (EPI == EPI_BIAS_GELU_D) {
        v += ld_v4(g.bias + n);
        float gv[4], gd[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pt_gelu_both_bf(v[i], gv[i], gd[i]);
        st_b4(g.C, c, floatx4{gd[0], gd[1], gd[2], gd[3]});
        st_b4(g.C2, (long)m * g.ldc2 + n, floatx4{gv[0], gv[1], gv[2], gv[3]});
    } else if (EPI == EPI_MUL) {
        st_b4(g.C, c, v * ld_b4(g.R, (long)m * g.ldr + n));
    } else if (EPI == EPI_BIAS_RESID) {
        st_b4(g.C, c, (v + ld_v4(g.bias + n)) + ld_v4(g.R + (long)m * g.ldr + n));
    }
}

// eight consecutive outputs C[m][n..n+7] (16 B bf16 stores; caller checked
// alignment and n + 7 < N); same arithmetic as epi_store4_bf
typedef __bf16 bf16x8s __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(1))) bf16x8s gbf16x8;
__device__ __forceinline__ void st_b8(float* base, long i, floatx4 a, floatx4 b) {
    *(gbf16x8*)(bfp(base) + i) = bf16x8s{(__bf16)a[0], (__bf16)a[1], (__bf16)a[2], (__bf16)a[3],
                                         (__bf16)b[0], (__bf16)b[1], (__bf16)b[2], (__bf16)b[3]};
}
template <int EPI>
__device__ __forceinline__ void epi_store8_bf(const GemmArgs& g, int m, int n, floatx4 v0, floatx4 v1) {
    const long c = (long)m * g.ldc + n;
    if (EPI == EPI_STORE) {
        st_b8(g.C, c, v0, v1);
    } else if (EPI == EPI_BIAS) {
        st_b8(g.C, c, v0 + ld_v4(g.bias + n), v1 + ld_v4(g.bias + n + 4));
    } else if (EPI == EPI_BIAS_GELU_D) {
        v0 += ld_v4(g.bias + n);
        v1 += ld_v4(g.bias + n + 4);
        float gv[8], gd[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pt_gelu_both_bf(v0[i], gv[i], gd[i]);
            pt_gelu_both_bf(v1[i], gv[4 + i], gd[4 + i]);
        }
        st_b8(g.C, c, floatx4{gd[0], gd[1], gd[2], gd[3]}, floatx4{gd[4], gd[5], gd[6], gd[7]});
        st_b8(g.C2, (long)m * g.ldc2 + n, floatx4{gv[0], gv[1], gv[2], gv[3]}, floatx4{gv[4], gv[5], gv[6], gv[7]});
    } else if (EPI == EPI_MUL) {
        const bf16x8s r = *(const gbf16x8*)(bfp(g.R) + (long)m * g.ldr + n);
        st_b8(g.C, c, v0 * floatx4{(float)r[0], (float)r[1], (float)r[2], (float)r[3]},
              v1 * floatx4{(float)r[4], (float)r[5], (float)r[6], (float)r[7]});
    } else if (EPI == EPI_BIAS_RESID) {
        st_b8(g.C, c, (v0 + ld_v4(g.bias + n)) + ld_v4(g.R + (long)m * g.ldr + n),
              (v1 + ld_v4(g.bias + n + 4)) + ld_v4(g.R + (long)m * g.ldr + n + 4));
    }
}

template <int EPI, bool OB = false>
__device__ __forceinline__ void epi_store4(const GemmArgs& g, int m, int n, floatx4 v) {
    if (OB) {
        epi_store4_bf<EPI>(g, m, n, v);
        return;
    }
    float* c = g.C + (long)m * g.ldc + n;
    if (EPI == EPI_STORE) {
        st_g4(c, v);
    } else if (EPI == EPI_BIAS) {
        st_g4(c, v + ld_v4(g.bias + n));
    } else if (EPI == EPI_BIAS_GELU) {
        v += ld_v4(g.bias + n);
        st_g4(c, v);
        st_g4(g.C2 + (long)m * g.ldc2 + n, floatx4{pt_gelu(v[0]), pt_gelu(v[1]), pt_gelu(v[2]), pt_gelu(v[3])});
    } else if (EPI == EPI_BIAS_RESID) {
        st_g4(c, (v + ld_v4(g.bias + n)) + ld_v4(g.R + (long)m * g.ldr + n));
    } else if (EPI == EPI_GELU_BWD) {
        const floatx4 x = ld_v4(g.R + (long)m * g.ldr + n);
        st_g4(c, v * floatx4{pt_gelu_grad(x[0]), pt_gelu_grad(x[1]), pt_gelu_grad(x[2]), pt_gelu_grad(x[3])});
    } else if (EPI == EPI_BIAS_GELU_D) {
        v += ld_v4(g.bias + n);
        float gv[4], gd[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pt_gelu_both(v[i], gv[i], gd[i]);
        st_g4(c, floatx4{gd[0], gd[1], gd[2], gd[3]});
        st_g4(g.C2 + (long)m * g.ldc2 + n, floatx4{gv[0], gv[1], gv[2], gv[3]});
    } else if (EPI == EPI_MUL) {
        st_g4(c, v * ld_v4(g.R + (long)m * g.ldr + n));
    } else if (EPI == EPI_AXPBY) {
        st_g4(c, g.alpha * v + g.beta * ld_v4(g.R + (long)m * g.ldr + n));
    } else if (EPI == EPI_ACCUM) {
        st_g4(c, ld_v4(c) + v);
    }
}

// fp32 store of an R-reading epilogue whose R segment r is already loaded.
template <int EPI>
__device__ __forceinline__ void epi_store4_r(const GemmArgs& g, int m, int n, floatx4 v, floatx4 r) {
    float* c = g.C + (long)m * g.ldc + n;
    if (EPI == EPI_BIAS_RESID) st_g4(c, (v + ld_v4(g.bias + n)) + r);
    else if (EPI == EPI_GELU_BWD)
        st_g4(c, v * floatx4{pt_gelu_grad(r[0]), pt_gelu_grad(r[1]), pt_gelu_grad(r[2]), pt_gelu_grad(r[3])});
    else if (EPI == EPI_MUL) st_g4(c, v * r);
    else if (EPI == EPI_AXPBY) st_g4(c, g.alpha * v + g.beta * r);
}

// Operand load of 4 consecutive floats along the contiguous dimension for
// shapes that break the 128-bit rules (a width or leading dimension not a
// multiple of 4, as the reference's 127-, 134- and 634-wide inputs do):
// scalar loads, each bounds-checked.  T: X[k][r..r+3], else X[r][k..k+3].
template <bool T>
__device__ __forceinline__ float4 ld_scalar4(const gfloat* X, long ld, int lim, int r, int k, int kend) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (T) {
        if (k < kend) {
            const gfloat* p = X + (long)k * ld + r;
            if (r < lim) v.x = p[0];
            if (r + 1 < lim) v.y = p[1];
            if (r + 2 < lim) v.z = p[2];
            if (r + 3 < lim) v.w = p[3];
        }
    } else if (r < lim) {
        const gfloat* p = X + (long)r * ld + k;
        if (k < kend) v.x = p[0];
        if (k + 1 < kend) v.y = p[1];
        if (k + 2 < kend) v.z = p[2];
        if (k + 3 < kend) v.w = p[3];
    }
    return v;
}

// Epilogues with a residual / pre-activation operand or the GELU: the tile
// goes through LDS in two 64-row halves and a rolled loop applies the
// epilogue to row-contiguous float4s (one GELU body instead of 64 inlined
// copies, whose code would not fit the instruction cache; R is read 512 B
// per row).  Staging layout [64][SST]; half h holds the rows
// wm + 32h .. wm + 32h + 31 of both wave rows.
constexpr int SST = BN + 4;
constexpr int STAGE_FLOATS = 64 * SST;
template <int EPI> struct EpiStaged {
    static constexpr bool value = EPI == EPI_BIAS_GELU || EPI == EPI_GELU_BWD || EPI == EPI_BIAS_RESID ||
                                  EPI == EPI_BIAS_GELU_D || EPI == EPI_MUL || EPI == EPI_AXPBY;
};

template <int EPI>
__device__ __forceinline__ void epilogue_staged(const GemmArgs& g, floatx4 (&acc)[4][4], int m0, int n0, int wm,
                                                int wn, int li, int lq, float* stage, bool vo) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        __syncthreads();   // the stage is free (main loop done / previous half consumed)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int tj = 0; tj < 4; ++tj)
                *reinterpret_cast<floatx4*>(stage + ((wm >> 6) * 32 + u * 16 + li) * SST + wn + tj * 16 + 4 * lq) =
                    acc[2 * h + u][tj];
        __syncthreads();
        for (int it = tid; it < 64 * (BN / 4); it += NT) {
            const int lr = it / (BN / 4), c = (it % (BN / 4)) * 4;
            const int m = m0 + (lr >> 5) * 64 + 32 * h + (lr & 31), n = n0 + c;
            if (m >= g.M || n >= g.N) continue;
            const floatx4 v = *reinterpret_cast<const floatx4*>(stage + lr * SST + c);
            if (vo && n + 3 < g.N) {
                epi_store4<EPI>(g, m, n, v);
            } else {
                for (int r = 0; r < 4 && n + r < g.N; ++r) epi_store<EPI>(g, m, n + r, v[r]);
            }
        }
    }
}

// 32 x 32 MFMA accumulators (the fp32 DMA tile's v_mfma_f32_32x32x2_f32 and
// the bf16-operand kernels' v_mfma_f32_32x32x16_bf16): with B as the first
// operand, register r of lane (l32 = lane % 32, lh = lane / 32) of acc[ti][tj]
// holds C[wm + 32 ti + l32][wn + 32 tj + 8 (r / 4) + 4 lh + r % 4] — four runs
// of four consecutive columns of one row.  The tile leaves through the LDS
// stage in two halves (half h = rows wm + 32 h .. + 31 of both wave rows) as
// row-contiguous float4s (bf16 outputs: eight columns per thread when vo8).
typedef float floatx16 __attribute__((ext_vector_type(16)));

// bf16 outputs (OB) are written eight columns per thread (16 B stores) when
// vo8: bases 16 B aligned and leading dimensions multiples of 8
template <int EPI, bool OB>
__device__ __forceinline__ void epilogue_staged32(const GemmArgs& g, floatx16 (&acc)[2][2], int m0, int n0, int wm,
                                                  int wn, int l32, int lh, float* stage, bool vo, bool vo8) {
    const int tid = threadIdx.x;
    // fp32 epilogues that read R load half of each row half's R segments
    // before that half's staging barriers and the rest right after them, so
    // the loads overlap the LDS round (all of them up front would cost a
    // fourth of the occupancy in registers).  The loads are branch-free: a
    // segment outside C reads R's first 4 floats and is not used.
    constexpr bool RPF = !OB && (EPI == EPI_BIAS_RESID || EPI == EPI_GELU_BWD || EPI == EPI_MUL || EPI == EPI_AXPBY);
    constexpr int RI = 64 * (BN / 4) / NT, RH = RI / 2;
    static_assert(64 * (BN / 4) % NT == 0, "epilogue segments must tile the threads");
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        floatx4 rv[RPF ? RI : 1];
        auto load_r = [&](int j) {
            const int it = tid + j * NT, lr = it / (BN / 4), c = (it % (BN / 4)) * 4;
            const int m = m0 + (lr >> 5) * 64 + 32 * h + (lr & 31), n = n0 + c;
            const bool ok = m < g.M && n + 3 < g.N;
            rv[j] = ld_v4(g.R + (ok ? (long)m * g.ldr + n : 0L));
        };
        if (RPF && vo) {
#pragma unroll
            for (int j = 0; j < RH; ++j) load_r(j);
        }
        __syncthreads();   // the stage is free (main loop done / previous half consumed)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<floatx4*>(stage + ((wm >> 6) * 32 + l32) * SST + wn + 32 * tj + 8 * q + 4 * lh) =
                    floatx4{acc[h][tj][4 * q], acc[h][tj][4 * q + 1], acc[h][tj][4 * q + 2], acc[h][tj][4 * q + 3]};
        __syncthreads();
        if (OB && vo8) {
            for (int it = tid; it < 64 * (BN / 8); it += NT) {
                const int lr = it / (BN / 8), c = (it % (BN / 8)) * 8;
                const int m = m0 + (lr >> 5) * 64 + 32 * h + (lr & 31), n = n0 + c;
                if (m >= g.M || n >= g.N) continue;
                const floatx4 v0 = *reinterpret_cast<const floatx4*>(stage + lr * SST + c);
                const floatx4 v1 = *reinterpret_cast<const floatx4*>(stage + lr * SST + c + 4);
                if (n + 7 < g.N) {
                    epi_store8_bf<EPI>(g, m, n, v0, v1);
                } else {
                    for (int r = 0; r < 4 && n + r < g.N; ++r) epi_store<EPI, OB>(g, m, n + r, v0[r]);
                    for (int r = 0; r < 4 && n + 4 + r < g.N; ++r) epi_store<EPI, OB>(g, m, n + 4 + r, v1[r]);
                }
            }
            continue;
        }
        if (RPF && vo) {
#pragma unroll
            for (int j = RH; j < RI; ++j) load_r(j);
#pragma unroll
            for (int j = 0; j < RI; ++j) {
                const int it = tid + j * NT, lr = it / (BN / 4), c = (it % (BN / 4)) * 4;
                const int m = m0 + (lr >> 5) * 64 + 32 * h + (lr & 31), n = n0 + c;
                if (m >= g.M || n >= g.N) continue;
                const floatx4 v = *reinterpret_cast<const floatx4*>(stage + lr * SST + c);
                if (n + 3 < g.N) epi_store4_r<EPI>(g, m, n, v, rv[j]);
                else
                    for (int r = 0; r < 4 && n + r < g.N; ++r) epi_store<EPI, OB>(g, m, n + r, v[r]);
            }
            continue;
        }
        for (int it = tid; it < 64 * (BN / 4); it += NT) {
            const int lr = it / (BN / 4), c = (it % (BN / 4)) * 4;
            const int m = m0 + (lr >> 5) * 64 + 32 * h + (lr & 31), n = n0 + c;
            if (m >= g.M || n >= g.N) continue;
            const floatx4 v = *reinterpret_cast<const floatx4*>(stage + lr * SST + c);
            if (vo && n + 3 < g.N) {
                epi_store4<EPI, OB>(g, m, n, v);
            } else {
                for (int r = 0; r < 4 && n + r < g.N; ++r) epi_store<EPI, OB>(g, m, n + r, v[r]);
            }
        }
    }
}


// Epilogue shared by the fp32 and bf16 kernels.  The MFMAs take the B tile
// as their first operand, so acc[ti][tj][r] holds the transposed product
// C[wm + ti*16 + li][wn + tj*16 + 4*lq + r] of the block tile at (m0, n0):
// four consecutive columns of one row per lane, stored (and the bias /
// residual / pre-activation read) as one 128-bit access when aligned.
// stage: STAGE_FLOATS of LDS the main loop no longer uses.
template <int EPI, bool PARTIAL>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g, floatx4 (&acc)[4][4], int m0, int n0, int wm,
                                              int wn, int li, int lq, long part_stride, float* stage, int bz) {
    if (PARTIAL && g.tail_part) {
        // tile-local partial [split][tile - tile0][BM][BN] (no bounds: the reduce masks)
        const int tn = (g.N + BN - 1) / BN;
        const long t = (long)(m0 / BM) * tn + n0 / BN - g.tile0;
        float* P = g.C + ((long)bz * g.ntiles + t) * (BM * BN);
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
#pragma unroll
            for (int tj = 0; tj < 4; ++tj) st_g4(P + (wm + ti * 16 + li) * BN + wn + tj * 16 + 4 * lq, acc[ti][tj]);
        return;
    }
    const long zoff = PARTIAL ? (long)bz * part_stride : 0;
    const uintptr_t al = PARTIAL ? (uintptr_t)g.C | (uintptr_t)(g.ldc * 4)
                                 : (uintptr_t)g.C | (uintptr_t)g.C2 | (uintptr_t)g.R | (uintptr_t)g.bias |
                                       (uintptr_t)((g.ldc | g.ldc2 | g.ldr) * 4);
    const bool vo = (al & 15) == 0;
    if (!PARTIAL && EpiStaged<EPI>::value) {
        epilogue_staged<EPI>(g, acc, m0, n0, wm, wn, li, lq, stage, vo);
        return;
    }
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
        const int m = m0 + wm + ti * 16 + li;
        if (m >= g.M) continue;
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) {
            const int n = n0 + wn + tj * 16 + 4 * lq;
            if (vo && n + 3 < g.N) {
                if (PARTIAL) st_g4(g.C + zoff + (long)m * g.ldc + n, acc[ti][tj]);
                else epi_store4<EPI>(g, m, n, acc[ti][tj]);
                continue;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (n + r >= g.N) continue;
                if (PARTIAL) g.C[zoff + (long)m * g.ldc + n + r] = acc[ti][tj][r];
                else epi_store<EPI>(g, m, n + r, acc[ti][tj][r]);
            }
        }
    }
}

// DB (AT only): blocks of the first N-tile also sum their A tile over k, the
// bias gradient sum_k dY[k][m]; thread t covers m = t % 128 over k half t / 128.
// With PARTIAL the per-split sums go to C + splits*part_stride + z*M.
// VEC: operands satisfy the 128-bit load rules (else scalar loads).
template <bool AT, bool BT, int EPI, bool PARTIAL, bool DB, bool VEC>
__global__ __launch_bounds__(NT) void gemm_f32_kernel(const GemmArgs g0, int k_chunk0, long part_stride) {
    const GemmArgs g = gemm_shape(g0);
    // a device reduction count splits its own K evenly over the launch's splits
    const int k_chunk = g0.Kdev ? (((g.K + (int)gridDim.z - 1) / (int)gridDim.z + BK - 1) / BK) * BK : k_chunk0;
    // one LDS array: the operand stages, reused by the staged epilogue
    constexpr int SMEM = 2 * (Stage<AT>::floats + Stage<BT>::floats);
    static_assert(SMEM >= STAGE_FLOATS, "epilogue stage does not fit the operand stages");
    __shared__ __align__(16) float smem[SMEM];
    float (*As)[Stage<AT>::floats] = reinterpret_cast<float (*)[Stage<AT>::floats]>(smem);
    float (*Bs)[Stage<BT>::floats] = reinterpret_cast<float (*)[Stage<BT>::floats]>(smem + 2 * Stage<AT>::floats);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tn = (g.N + BN - 1) / BN;
    int tmi, tni;
    if (!tile_of_range(g, tn, tmi, tni, blockIdx.x)) return;   // beyond the (device) tile count
    const int m0 = tmi * BM, n0 = tni * BN;
    const int kbeg = blockIdx.z * k_chunk;
    const int kend = min(g.K, kbeg + k_chunk);
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int li = lane & 15, lq = lane >> 4;

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // operands are global memory: say so, or the loads become flat loads that
    // also count against lgkmcnt and stall the LDS waits on global latency
    const gfloat* __restrict__ Ag = (const gfloat*)(g.A);
    const gfloat* __restrict__ Bg = (const gfloat*)(g.B);
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    // per-thread staging slots: 128 rows x 16 k = 512 float4 per operand, two per thread
    // (T == false: row idx>>2, k quarter idx&3; T == true: k row idx>>5, 4-row group idx&31)
    const int i0 = tid, i1 = tid + NT;
    const int ra0 = AT ? (i0 & 31) * 4 : (i0 >> 2), rk0 = AT ? (i0 >> 5) : (i0 & 3) * 4;
    const int ra1 = AT ? (i1 & 31) * 4 : (i1 >> 2), rk1 = AT ? (i1 >> 5) : (i1 & 3) * 4;
    const int rb0 = BT ? (i0 & 31) * 4 : (i0 >> 2), kb0 = BT ? (i0 >> 5) : (i0 & 3) * 4;
    const int rb1 = BT ? (i1 & 31) * 4 : (i1 >> 2), kb1 = BT ? (i1 >> 5) : (i1 & 3) * 4;
    const int sa0 = AT ? rk0 * SM + ra0 : ra0 * SK + rk0, sa1 = AT ? rk1 * SM + ra1 : ra1 * SK + rk1;
    const int sb0 = BT ? kb0 * SM + rb0 : rb0 * SK + kb0, sb1 = BT ? kb1 * SM + rb1 : rb1 * SK + kb1;
#define PT_LD(X, ld, lim, r0, T, rr, kk, k0)                                                   \
    (!VEC ? ld_scalar4<T>((X), (ld), (lim), (r0) + (rr), (k0) + (kk), kend)                      \
     : ((r0) + (rr) < (lim) && (k0) + (kk) < kend)                                              \
         ? ld_g4((X) + ((T) ? (long)((k0) + (kk)) * (ld) + (r0) + (rr)                       \
                            : (long)((r0) + (rr)) * (ld) + (k0) + (kk)))                        \
         : z4)
    float4 va0, va1, vb0, vb1;
#define PT_GLOAD(k0)                                           \
    va0 = PT_LD(Ag, g.lda, g.M, m0, AT, ra0, rk0, k0);         \
    va1 = PT_LD(Ag, g.lda, g.M, m0, AT, ra1, rk1, k0);         \
    vb0 = PT_LD(Bg, g.ldb, g.N, n0, BT, rb0, kb0, k0);         \
    vb1 = PT_LD(Bg, g.ldb, g.N, n0, BT, rb1, kb1, k0);
#define PT_SSTORE(buf)                                         \
    *reinterpret_cast<float4*>(&As[buf][sa0]) = va0;           \
    *reinterpret_cast<float4*>(&As[buf][sa1]) = va1;           \
    *reinterpret_cast<float4*>(&Bs[buf][sb0]) = vb0;           \
    *reinterpret_cast<float4*>(&Bs[buf][sb1]) = vb1;

    const bool do_db = DB && AT && tni == 0;
    float dbsum = 0.f;
    if (kbeg < kend) {
        PT_GLOAD(kbeg)
        PT_SSTORE(0)
        __syncthreads();
        int buf = 0;
        for (int k0 = kbeg; k0 < kend; k0 += BK) {
            const bool more = k0 + BK < kend;
            if (more) { PT_GLOAD(k0 + BK) }
            const float* Ab = As[buf];
            const float* Bb = Bs[buf];
            float4 af[4], bf[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (!AT) af[t] = *reinterpret_cast<const float4*>(Ab + (wm + t * 16 + li) * SK + 4 * lq);
                else af[t] = make_float4(Ab[(4 * lq + 0) * SM + wm + t * 16 + li], Ab[(4 * lq + 1) * SM + wm + t * 16 + li],
                                         Ab[(4 * lq + 2) * SM + wm + t * 16 + li], Ab[(4 * lq + 3) * SM + wm + t * 16 + li]);
                if (!BT) bf[t] = *reinterpret_cast<const float4*>(Bb + (wn + t * 16 + li) * SK + 4 * lq);
                else bf[t] = make_float4(Bb[(4 * lq + 0) * SM + wn + t * 16 + li], Bb[(4 * lq + 1) * SM + wn + t * 16 + li],
                                         Bb[(4 * lq + 2) * SM + wn + t * 16 + li], Bb[(4 * lq + 3) * SM + wn + t * 16 + li]);
            }
#define PT_MFMA_STEP(c)                                                                             \
            _Pragma("unroll") for (int ti = 0; ti < 4; ++ti)                                        \
            _Pragma("unroll") for (int tj = 0; tj < 4; ++tj)                                        \
                acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[tj].c, af[ti].c, acc[ti][tj], 0, 0, 0);
            PT_MFMA_STEP(x) PT_MFMA_STEP(y) PT_MFMA_STEP(z) PT_MFMA_STEP(w)
#undef PT_MFMA_STEP
            if (do_db) {
                // rows beyond kend / columns beyond M were staged as zeros
#pragma unroll
                for (int kk = 0; kk < BK / 2; ++kk) dbsum += Ab[((tid >> 7) * (BK / 2) + kk) * SM + (tid & 127)];
            }
            if (more) { PT_SSTORE(buf ^ 1) }
            __syncthreads();
            buf ^= 1;
        }
    }
#undef PT_GLOAD
#undef PT_SSTORE
#undef PT_LD

    if (do_db) {
        // the loop ended on a barrier, so buffer 0 is free; fixed-order pair sum
        float* sh = As[0];
        sh[tid] = dbsum;
        __syncthreads();
        const int m = m0 + tid;
        if (tid < 128 && m < g.M) {
            const float v = sh[tid] + sh[tid + 128];
            if (PARTIAL) g.C[(long)gridDim.z * part_stride + (long)blockIdx.z * g.M + m] = v;
            else g.dbias[m] = v;
        }
    }

    gemm_epilogue<EPI, PARTIAL>(g, acc, m0, n0, wm, wn, li, lq, part_stride, smem, blockIdx.z);
}


// ---------------------------------------------------------------- fp32, LDS DMA
// Operand tiles go global -> LDS with buffer_load ... lds (16 B per lane;
// lane L writes L*16 B past the wave's LDS base), DMA_NS stages deep: no
// staging registers, and the loads of tile i + DMA_NS - 1 are in flight
// while tile i is multiplied.  Buffer loads return zero past the operand's
// last element (num_records = its exact extent), which zeroes the k tail of
// an m-contiguous operand; a k-contiguous operand's row tails (K % BK != 0)
// read the next row and are zeroed in LDS before the last tile's products.
// Rows / columns past M / N read what lies
// there or zero and only reach C rows / columns that are never stored.
// The DMA is issued from inline assembly so the compiler does not tie LDS
// reads to the outstanding loads; the loop waits on vmcnt itself.
constexpr int DMA_NS = 2;
typedef int int32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int32x4_t buffer_rsrc(const float* p, unsigned bytes) {
    const unsigned long long a = (unsigned long long)p;
    // uniform by construction; readfirstlane makes that explicit for operands
    // loaded from memory (the grouped launch's descriptors)
    int32x4_t r;
    r.x = __builtin_amdgcn_readfirstlane((int)(unsigned)(a & 0xffffffffull));
    r.y = __builtin_amdgcn_readfirstlane((int)(unsigned)(a >> 32));   // stride 0 (addresses are below 2^48)
    r.z = __builtin_amdgcn_readfirstlane((int)bytes);                 // num_records: bytes from the base
    r.w = 0x00020000;                 // gfx9 raw buffer: 32-bit data format, no swizzle
    return r;
}
__device__ __forceinline__ void dma16(int32x4_t rsrc, const float* lds_base, int voffset_bytes) {
    const unsigned lds = (unsigned)(uintptr_t)lds_base;   // LDS offset (low bits of the generic address)
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset_bytes), "s"(rsrc) : "memory", "m0");
}
template <int N> __device__ __forceinline__ void wait_vm() {
    static_assert(N % 4 == 0 && N <= 24, "wait_vm: 4 loads per stage, at most 6 later stages");
    if (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (N == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else if (N == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if (N == 20) asm volatile("s_waitcnt vmcnt(20)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
}
// wait until at most `later` stages (4 loads each) are still in flight
template <int NS> __device__ __forceinline__ void wait_stages(int later) {
    if (NS > 7 && later >= 6) wait_vm<24>();
    else if (NS > 6 && later == 5) wait_vm<20>();
    else if (NS > 5 && later == 4) wait_vm<16>();
    else if (NS > 4 && later == 3) wait_vm<12>();
    else if (NS > 3 && later == 2) wait_vm<8>();
    else if (NS > 2 && later == 1) wait_vm<4>();
    else wait_vm<0>();
}
// row swizzle of the [row][k] layout: conflict-free 128-bit reads of 16 rows
// (one k group) on 32- and 64-bank LDS, and conflict-free DMA writes
__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }
// DMA LDS layouts (unpadded, 4-float groups XOR-swizzled):
//   [row][k] (k-contiguous): element (r, k) at r*BK + 4*((k>>2) ^ swz(r)) + (k&3)
//   [k][row] (m-contiguous): element (k, r) at k*BM + 4*((r>>2) ^ (k&4)) + (r&3)
// The [row][k] swizzle keeps the fragment reads (16 rows, one group) on
// distinct banks; the [k][row] one puts the four k rows of a fragment read
// (k = 4*lq + c) on alternating bank halves.
template <bool T> __device__ __forceinline__ int dma_at(int r, int k) {
    return T ? k * BM + 4 * ((r >> 2) ^ (k & 4)) + (r & 3) : r * BK + 4 * ((k >> 2) ^ swz(r)) + (k & 3);
}
// Thread's chunk offset (elements, without the tile's k0) for DMA chunk c of
// a 128 x 16 operand tile: [row][k] chunk = rows 16c.., [k][row] chunk = k rows 2c, 2c+1
template <bool T> __device__ __forceinline__ int dma_src(int c, int lane, int r0, long ld) {
    if (!T) {
        const int r = 16 * c + (lane >> 2), gq = lane & 3;
        return (int)((r0 + r) * ld) + 4 * (gq ^ swz(r));
    }
    const int k = 2 * c + (lane >> 5), gq = lane & 31;
    return (int)(k * ld) + r0 + 4 * (gq ^ (k & 4));
}

// One 128 x 128 tile of C (split bz of gz along K) of the logical tile
// index bx; shared by the per-product launch and the grouped launch.
// NS: pipeline stages (NS - 1 tiles in flight while one is multiplied).
// fp32 products: a wave's 64 x 64 tile is 2 x 2 tiles of
// v_mfma_f32_32x32x2_f32 (153.6 TFLOP/s measured on this GPU against 139.6
// for the 16 x 16 x 4 form, with half the instructions): at step s (0..7) of
// a 16-k stage, lane (l32, lh) supplies row l32 of its 32-row slice at
// k = 8 lh + s for both A and B, so a k-contiguous ([row][k]) operand's
// eight values are two 128-bit LDS reads; the tile leaves through the
// 32 x 32 staged epilogue (row-contiguous stores).
// BF: bf16 products on 16 x 16 tiles — each lane's float4 fragment
// (k = 4 lq .. 4 lq + 3 of its row, the same k for A and B) is rounded to
// bf16 (RNE) and one v_mfma_f32_16x16x16_bf16 replaces four fp32 k-steps.
// LDS floats of an NS-stage DMA tile (operand stages, or the staged epilogue)
template <int NS> constexpr int dma_smem_floats() {
    return NS * 2 * BM * BK > STAGE_FLOATS ? NS * 2 * BM * BK : STAGE_FLOATS;
}
// smem: the calling kernel's LDS array of dma_smem_floats<NS>() floats (one
// array, so a kernel calling several forms of the tile holds it once)
template <bool AT, bool BT, int EPI, bool PARTIAL, bool DB, bool BF = false, int NS = DMA_NS>
__device__ __forceinline__ void gemm_dma_tile(const GemmArgs& g0, int k_chunk0, long part_stride, int bx, int bz,
                                              int gz, float* smem) {
    constexpr bool W32 = !BF;
    const GemmArgs g = gemm_shape(g0);
    // a device reduction count splits its own K evenly over the launch's
    // splits, or (wsplit) as many ways as the weight-gradient rule gives for
    // that count: the later splits return, and workgroup (0, 0, 0) leaves the
    // count after the partials (and bias partials) for the reduce
    int k_chunk = g0.Kdev ? (((g.K + gz - 1) / gz + BK - 1) / BK) * BK : k_chunk0;
    if constexpr (PARTIAL) {
        if (g0.Kdev && g0.wsplit) {
            const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
            const int sp = pt_split_chunks(g.K, min(pt_wgrad_splits(g.K, tiles, g0.wsplit, BK), gz), BK, &k_chunk);
            if (bx == 0 && bz == 0 && threadIdx.x == 0)
                *reinterpret_cast<int*>(g0.C + (long)gz * (part_stride + (DB ? g0.M : 0))) = sp;
            if (bz >= sp) return;
        }
    }
    constexpr int TILE = BM * BK;   // floats per operand tile (BM == BN)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tn = (g.N + BN - 1) / BN;
    int tmi, tni;
    if (!tile_of_range(g, tn, tmi, tni, bx)) return;   // beyond the tile count
    const int m0 = tmi * BM, n0 = tni * BN;
    const int kbeg = bz * k_chunk;
    const int kend = min(g.K, kbeg + k_chunk);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int li = lane & 15, lq = lane >> 4;
    const int l32 = lane & 31, lh = lane >> 5;

    floatx4 acc[4][4];       // 16 x 16 tiles (BF)
    floatx16 acc32[2][2];    // 32 x 32 tiles (fp32)
    if constexpr (W32) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc32[i][j][e] = 0.f;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

    // exact operand extents (host checked < 2^31 bytes)
    const unsigned ea = (unsigned)(AT ? ((long)(g.K - 1) * g.lda + g.M) : ((long)(g.M - 1) * g.lda + g.K)) * 4u;
    const unsigned eb = (unsigned)(BT ? ((long)(g.K - 1) * g.ldb + g.N) : ((long)(g.N - 1) * g.ldb + g.K)) * 4u;
    const int32x4_t ra = buffer_rsrc(g.A, ea), rb = buffer_rsrc(g.B, eb);
    const int sa0 = dma_src<AT>(2 * wave, lane, m0, g.lda), sa1 = dma_src<AT>(2 * wave + 1, lane, m0, g.lda);
    const int sb0 = dma_src<BT>(2 * wave, lane, n0, g.ldb), sb1 = dma_src<BT>(2 * wave + 1, lane, n0, g.ldb);
    const int ka = AT ? (int)g.lda : 1, kb = BT ? (int)g.ldb : 1;   // element step per k
#define PT_ISSUE(tile)                                                                  \
    {                                                                                   \
        const int k0_ = kbeg + (tile) * BK;                                             \
        const float* st_ = smem + ((tile) % NS) * 2 * TILE;                             \
        dma16(ra, st_ + (2 * wave) * 256, (sa0 + k0_ * ka) * 4);                        \
        dma16(ra, st_ + (2 * wave + 1) * 256, (sa1 + k0_ * ka) * 4);                    \
        dma16(rb, st_ + TILE + (2 * wave) * 256, (sb0 + k0_ * kb) * 4);                 \
        dma16(rb, st_ + TILE + (2 * wave + 1) * 256, (sb1 + k0_ * kb) * 4);             \
    }
    const bool do_db = DB && AT && tni == 0;
    float dbsum = 0.f;
    if (nk > 0) {
#pragma unroll
        for (int t = 0; t < NS - 1; ++t)
            if (t < nk) PT_ISSUE(t)
        for (int it = 0; it < nk; ++it) {
            // tile it has landed once at most min(NS - 2, nk - 1 - it) later
            // tiles (4 loads each) are still in flight
            wait_stages<NS>(min(NS - 2, nk - 1 - it));
            __syncthreads();   // every wave's loads of tile it are in LDS; tile it - 1 is consumed
            if (!(AT && BT)) {
                // the product's last tile may end inside the stage (K % 16 != 0):
                // a k-contiguous operand's DMA also brought the floats past each
                // row's end (the next row, or zeros past the extent) — zero those
                // k columns before the products
                const int kv = kend - (kbeg + it * BK);
                if (kv < BK) {
                    float* st = smem + (it % NS) * 2 * TILE;
                    for (int idx = tid; idx < BM * BK; idx += NT) {
                        const int r = idx / BK, k = idx % BK;
                        if (k >= kv) {
                            if (!AT) st[dma_at<false>(r, k)] = 0.f;
                            if (!BT) st[TILE + dma_at<false>(r, k)] = 0.f;
                        }
                    }
                    __syncthreads();
                }
            }
            if (it + NS - 1 < nk) PT_ISSUE(it + NS - 1)
            const float* Ab = smem + (it % NS) * 2 * TILE;
            const float* Bb = Ab + TILE;
            if constexpr (W32) {
                // lane (l32, lh): rows wm / wn + 32 t + l32, k = 8 lh .. 8 lh + 7
                float a8[2][8], b8[2][8];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int ca = wm + 32 * t + l32, cb = wn + 32 * t + l32;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int k0 = 8 * lh + 4 * h;
                        float4 va, vb;
                        if (!AT) va = *reinterpret_cast<const float4*>(Ab + dma_at<false>(ca, k0));
                        else va = make_float4(Ab[dma_at<true>(ca, k0)], Ab[dma_at<true>(ca, k0 + 1)],
                                              Ab[dma_at<true>(ca, k0 + 2)], Ab[dma_at<true>(ca, k0 + 3)]);
                        if (!BT) vb = *reinterpret_cast<const float4*>(Bb + dma_at<false>(cb, k0));
                        else vb = make_float4(Bb[dma_at<true>(cb, k0)], Bb[dma_at<true>(cb, k0 + 1)],
                                              Bb[dma_at<true>(cb, k0 + 2)], Bb[dma_at<true>(cb, k0 + 3)]);
                        a8[t][4 * h] = va.x; a8[t][4 * h + 1] = va.y; a8[t][4 * h + 2] = va.z; a8[t][4 * h + 3] = va.w;
                        b8[t][4 * h] = vb.x; b8[t][4 * h + 1] = vb.y; b8[t][4 * h + 2] = vb.z; b8[t][4 * h + 3] = vb.w;
                    }
                }
#pragma unroll
                for (int st = 0; st < 8; ++st)
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int tj = 0; tj < 2; ++tj)
                            acc32[ti][tj] =
                                __builtin_amdgcn_mfma_f32_32x32x2f32(b8[tj][st], a8[ti][st], acc32[ti][tj], 0, 0, 0);
                if (do_db) {
                    // k rows past K were loaded as zeros; columns past M are never stored
#pragma unroll
                    for (int kk = 0; kk < BK / 2; ++kk)
                        dbsum += Ab[dma_at<true>(tid & 127, (tid >> 7) * (BK / 2) + kk)];
                }
                continue;
            }
            float4 af[4], bf[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int ca = wm + t * 16 + li, cb = wn + t * 16 + li;
                if (!AT) af[t] = *reinterpret_cast<const float4*>(Ab + dma_at<false>(ca, 4 * lq));
                else af[t] = make_float4(Ab[dma_at<true>(ca, 4 * lq)], Ab[dma_at<true>(ca, 4 * lq + 1)],
                                         Ab[dma_at<true>(ca, 4 * lq + 2)], Ab[dma_at<true>(ca, 4 * lq + 3)]);
                if (!BT) bf[t] = *reinterpret_cast<const float4*>(Bb + dma_at<false>(cb, 4 * lq));
                else bf[t] = make_float4(Bb[dma_at<true>(cb, 4 * lq)], Bb[dma_at<true>(cb, 4 * lq + 1)],
                                         Bb[dma_at<true>(cb, 4 * lq + 2)], Bb[dma_at<true>(cb, 4 * lq + 3)]);
            }
            if constexpr (BF) {
                bf16x4 ah[4], bh[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    ah[t] = to_bf16x4(af[t].x, af[t].y, af[t].z, af[t].w);
                    bh[t] = to_bf16x4(bf[t].x, bf[t].y, bf[t].z, bf[t].w);
                }
#pragma unroll
                for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                    for (int tj = 0; tj < 4; ++tj)
                        acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bh[tj], ah[ti], acc[ti][tj], 0, 0, 0);
            } else {
#define PT_MFMA_STEP(c)                                                                             \
            _Pragma("unroll") for (int ti = 0; ti < 4; ++ti)                                        \
            _Pragma("unroll") for (int tj = 0; tj < 4; ++tj)                                        \
                acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[tj].c, af[ti].c, acc[ti][tj], 0, 0, 0);
            PT_MFMA_STEP(x) PT_MFMA_STEP(y) PT_MFMA_STEP(z) PT_MFMA_STEP(w)
#undef PT_MFMA_STEP
            }
            if (do_db) {
                // k rows past K were loaded as zeros; columns past M are never stored
#pragma unroll
                for (int kk = 0; kk < BK / 2; ++kk) dbsum += Ab[dma_at<true>(tid & 127, (tid >> 7) * (BK / 2) + kk)];
            }
        }
    }
#undef PT_ISSUE
    __syncthreads();   // the stages are free for the bias sums / staged epilogue

    if (do_db) {
        float* sh = smem;
        sh[tid] = dbsum;
        __syncthreads();
        const int m = m0 + tid;
        if (tid < 128 && m < g.M) {
            const float v = sh[tid] + sh[tid + 128];
            if (PARTIAL) g.C[(long)gz * part_stride + (long)bz * g.M + m] = v;
            else g.dbias[m] = v;
        }
    }

    if constexpr (W32) {
        if (PARTIAL && g.tail_part) {
            // tile-local partial [split][tile - tile0][BM][BN] (no bounds: the reduce masks)
            const long t = (long)tmi * tn + tni - g.tile0;
            float* P = g.C + ((long)bz * g.ntiles + t) * (BM * BN);
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                for (int tj = 0; tj < 2; ++tj)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        st_g4(P + (wm + 32 * ti + l32) * BN + wn + 32 * tj + 8 * q + 4 * lh,
                              floatx4{acc32[ti][tj][4 * q], acc32[ti][tj][4 * q + 1], acc32[ti][tj][4 * q + 2],
                                      acc32[ti][tj][4 * q + 3]});
            return;
        }
        GemmArgs ge = g;
        if (PARTIAL) ge.C = g.C + (long)bz * part_stride;   // split-K partial: a plain store
        const uintptr_t al = PARTIAL ? (uintptr_t)ge.C | (uintptr_t)(g.ldc * 4)
                                     : (uintptr_t)g.C | (uintptr_t)g.C2 | (uintptr_t)g.R | (uintptr_t)g.bias |
                                           (uintptr_t)((g.ldc | g.ldc2 | g.ldr) * 4);
        const bool vo = (al & 15) == 0;
        if (PARTIAL || !EpiStaged<EPI>::value) {
            // plain, bias and accumulate outputs straight from the accumulators:
            // a store instruction covers 32 rows x 32 B, and the wave's four
            // stores of a run (8 q + 4 lh) fill each row's 128 B segment
            constexpr int E = PARTIAL ? EPI_STORE : EPI;
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                const int m = m0 + wm + 32 * ti + l32;
                if (m >= g.M) continue;
#pragma unroll
                for (int tj = 0; tj < 2; ++tj)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int n = n0 + wn + 32 * tj + 8 * q + 4 * lh;
                        const floatx4 v = floatx4{acc32[ti][tj][4 * q], acc32[ti][tj][4 * q + 1],
                                                  acc32[ti][tj][4 * q + 2], acc32[ti][tj][4 * q + 3]};
                        if (vo && n + 3 < g.N) {
                            epi_store4<E>(ge, m, n, v);
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (n + r < g.N) epi_store<E>(ge, m, n + r, v[r]);
                        }
                    }
            }
            return;
        }
        epilogue_staged32<EPI, false>(ge, acc32, m0, n0, wm, wn, l32, lh, smem, vo, false);
        return;
    }
    gemm_epilogue<EPI, PARTIAL>(g, acc, m0, n0, wm, wn, li, lq, part_stride, smem, bz);
}

template <bool AT, bool BT, int EPI, bool PARTIAL, bool DB>
__global__ __launch_bounds__(NT) void gemm_f32_dma_kernel(const GemmArgs g0, int k_chunk0, long part_stride) {
    __shared__ __align__(16) float smem[dma_smem_floats<DMA_NS>()];
    gemm_dma_tile<AT, BT, EPI, PARTIAL, DB>(g0, k_chunk0, part_stride, blockIdx.x, blockIdx.z, gridDim.z, smem);
}

// The balanced last wave of pt_gemm's host-count launches, decided from a
// device row count: with T tiles on S CUs and R = T % S tail tiles (when
// S < T < 4 S and at least two k-splits fit per tail tile), tiles [0, T - R)
// run whole and the R tail tiles split K s2 = S / R ways (chunks of kc,
// rounded to the k-step), their partials tile-local in the workspace.  The
// same arithmetic as the host's, so the same tiles, splits and sums.
struct DTail {
    int full, R, s2, kc;
};
__device__ __forceinline__ DTail dtail_plan(const GemmArgs& g, int S) {
    const int count = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    const int ksteps = (g.K + BK - 1) / BK;
    DTail p{count, 0, 1, g.K};
    const int R = count % S;
    int s2 = R ? S / R : 0;
    if (s2 > ksteps / 2) s2 = ksteps / 2;
    if (count > S && count < 4 * S && R != 0 && s2 >= 2) {
        p.kc = (((g.K + s2 - 1) / s2 + BK - 1) / BK) * BK;
        p.s2 = (g.K + p.kc - 1) / p.kc;
        p.R = R;
        p.full = count - R;
    }
    return p;
}

// A device-row-count product with its last wave balanced: workgroups
// [0, full) take whole tiles (epilogue applied), the next R s2 take split
// u / R of tail tile u % R (partials into part); the rest of the launch
// (sized for the host's row bound plus one workgroup per CU) returns.
// dtail_reduce_kernel sums the partials after it: the kernel boundary makes
// them visible to every XCD, where a reduction by the last split to arrive
// would need an agent-scope release per tail workgroup (an L2 write-back on
// this GPU, measured slower than the unbalanced wave).
template <bool AT, bool BT, int EPI>
__global__ __launch_bounds__(NT) void gemm_f32_dma_dtail_kernel(const GemmArgs g0, float* __restrict__ part,
                                                               int S) {
    __shared__ __align__(16) float smem[dma_smem_floats<DMA_NS>()];
    const DTail p = dtail_plan(gemm_shape(g0), S);
    const int b = blockIdx.x;
    if (b < p.full) {
        GemmArgs f = g0;
        f.tile0 = 0;
        f.ntiles = p.full;
        gemm_dma_tile<AT, BT, EPI, false, false>(f, g0.K, 0, b, 0, 1, smem);
        return;
    }
    const int u = b - p.full;
    if (u >= p.R * p.s2) return;
    GemmArgs q = g0;
    q.C = part;
    q.tile0 = p.full;
    q.ntiles = p.R;
    q.tail_part = 1;
    gemm_dma_tile<AT, BT, EPI, true, false>(q, p.kc, 0, u % p.R, u / p.R, p.s2, smem);
}

// The tail tiles of gemm_f32_dma_dtail_kernel: 16 workgroups per tail tile
// (tile-major, so the launch's S * 16 workgroups past R * 16 return), each
// thread one float4 of tile t: its s2 partials summed in split order through
// the epilogue (tail_reduce_kernel's arithmetic, the plan taken from the
// device row count).
constexpr int DTAIL_RED_WG = BM * BN / 4 / 256;
template <int EPI>
__global__ __launch_bounds__(256) void dtail_reduce_kernel(const GemmArgs g0, const float* __restrict__ part,
                                                           int S) {
    const GemmArgs g = gemm_shape(g0);
    const DTail p = dtail_plan(g, S);
    const int t = blockIdx.x / DTAIL_RED_WG;
    if (t >= p.R) return;
    const int tn = (g.N + BN - 1) / BN, lt = p.full + t;
    const int m0 = (lt / tn) * BM, n0 = (lt % tn) * BN;
    {
        const int e = 4 * ((blockIdx.x % DTAIL_RED_WG) * 256 + threadIdx.x);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int z = 0; z < p.s2; ++z) {
            const float4 w = *reinterpret_cast<const float4*>(part + ((long)z * p.R + t) * (BM * BN) + e);
            v.x += w.x;
            v.y += w.y;
            v.z += w.z;
            v.w += w.w;
        }
        const int m = m0 + e / BN, n = n0 + e % BN;
        if (m < g.M) {
            if (n < g.N) epi_store<EPI>(g, m, n, v.x);
            if (n + 1 < g.N) epi_store<EPI>(g, m, n + 1, v.y);
            if (n + 2 < g.N) epi_store<EPI>(g, m, n + 2, v.z);
            if (n + 3 < g.N) epi_store<EPI>(g, m, n + 3, v.w);
        }
    }
}

// ---------------------------------------------------------------- residual + LayerNorm
// C = A W^T + bias + R (a pre-LN block's residual add, EPI_BIAS_RESID) at
// N = 256, followed in the same launch by the LayerNorm of C's rows that the
// next stage reads: Y = LN(C) lnw + lnb with its mean and rstd.  The unfused
// pair is the DMA kernel's EPI_BIAS_RESID then ln_fwd_kernel, which reads C
// back from HBM.  A workgroup owns BMR (64 or 32) full rows: a BMR x 256
// tile, the four waves side by side, each a BMR x 64 sub-tile of
// v_mfma_f32_32x32x2_f32 tiles (2 x 2 or 1 x 2) with the DMA kernel's operand
// order, so every output accumulates the same products in the same order.  Per 16-k stage
// the A rows (one 16-row chunk) and W rows (four chunks) go global -> LDS by
// DMA, two stages deep.  The tile leaves through LDS in 32-row halves; a
// wave then takes eight rows, one float4 per lane, adds bias and residual in
// epi_store4_r's order and normalises in ln_fwd_kernel's order (two-pass
// mean / variance by wave sums, eps 1e-5), so C, Y, mean and rstd equal the
// unfused pair's bit for bit.  K % 16 == 0, N = 256 (host checked).
// BF: A and W hold bf16 (the mixed-precision variant's activations and weight
// copies; K, lda, ldb in float units, 2 bf16 per float) and the products run
// on v_mfma_f32_32x32x16_bf16 in gemm_bs32_kernel's fragment order; YB: Y is
// stored in bf16 (round to nearest even), ldy in bf16 elements.
constexpr int RL_BM = 64, RL_N = 256, RL_SST = RL_N + 4;
template <bool BF, bool YB, int BMR = RL_BM>
__global__ __launch_bounds__(NT) void gemm_resid_ln_kernel(const GemmArgs g0, const float* __restrict__ lnw,
        const float* __restrict__ lnb, float* __restrict__ Y, long ldy, float* __restrict__ mean,
        float* __restrict__ rstd) {
    const GemmArgs g = gemm_shape(g0);
    static_assert(BMR == 128 || BMR == 64 || BMR == 32, "128-, 64- or 32-row tiles");
    static_assert(BF || BMR <= 64, "fp32 operands: 64- or 32-row tiles");
    constexpr int TM = BMR / 32;   // 32-row MFMA tiles per wave
    const int m0 = blockIdx.x * BMR;
    if (m0 >= g.M) return;   // beyond the (device) row count
    constexpr int TA = BMR * BK, TB = RL_N * BK, STAGE = TA + TB;
    constexpr int SMEM = 2 * STAGE > 32 * RL_SST ? 2 * STAGE : 32 * RL_SST;
    __shared__ __align__(16) float smem[SMEM];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, lh = lane >> 5;
    const int wn = 64 * wave;
    floatx16 acc[TM][2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    // exact operand extents (host checked < 2^31 bytes): rows past M read zeros
    const unsigned ea = (unsigned)(((long)(g.M - 1) * g.lda + g.K) * 4);
    const unsigned eb = (unsigned)(((long)(RL_N - 1) * g.ldb + g.K) * 4);
    const int32x4_t ra = buffer_rsrc(g.A, ea), rb = buffer_rsrc(g.B, eb);
    // A's 16-row chunks: chunk wave (and wave + 4 for 128-row tiles)
    const int sa = dma_src<false>(wave, lane, m0, g.lda), sa2 = dma_src<false>(wave + 4, lane, m0, g.lda);
    int sb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sb[j] = dma_src<false>(4 * wave + j, lane, 0, g.ldb);
    auto issue = [&](int tile) {
        const int k0 = tile * BK;
        const float* st = smem + (tile & 1) * STAGE;
        if (wave < BMR / 16) dma16(ra, st + wave * 256, (sa + k0) * 4);
        if (BMR == 128) dma16(ra, st + (wave + 4) * 256, (sa2 + k0) * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16(rb, st + TA + (4 * wave + j) * 256, (sb[j] + k0) * 4);
    };
    const int nk = g.K / BK;
    issue(0);
    for (int it = 0; it < nk; ++it) {
        wait_vm<0>();      // this wave's loads of tile it have landed
        __syncthreads();   // every wave's have; tile it - 1 is consumed
        if (it + 1 < nk) issue(it + 1);
        const float* Ab = smem + (it & 1) * STAGE;
        const float* Bb = Ab + TA;
        if constexpr (BF) {
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                bf16x8 ah[TM], bh[2];
#pragma unroll
                for (int t = 0; t < TM; ++t)
                    ah[t] = *reinterpret_cast<const bf16x8*>(Ab + dma_at<false>(32 * t + l32, 4 * (2 * st + lh)));
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    bh[t] = *reinterpret_cast<const bf16x8*>(Bb + dma_at<false>(wn + 32 * t + l32, 4 * (2 * st + lh)));
#pragma unroll
                for (int ti = 0; ti < TM; ++ti)
#pragma unroll
                    for (int tj = 0; tj < 2; ++tj)
                        acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh[tj], ah[ti], acc[ti][tj], 0, 0, 0);
            }
            continue;
        }
        float a8[TM][8], b8[2][8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int k0 = 8 * lh + 4 * h;
                if (t < TM) {
                    const float4 va = *reinterpret_cast<const float4*>(Ab + dma_at<false>(32 * t + l32, k0));
                    a8[t][4 * h] = va.x; a8[t][4 * h + 1] = va.y; a8[t][4 * h + 2] = va.z; a8[t][4 * h + 3] = va.w;
                }
                const float4 vb = *reinterpret_cast<const float4*>(Bb + dma_at<false>(wn + 32 * t + l32, k0));
                b8[t][4 * h] = vb.x; b8[t][4 * h + 1] = vb.y; b8[t][4 * h + 2] = vb.z; b8[t][4 * h + 3] = vb.w;
            }
#pragma unroll
        for (int st = 0; st < 8; ++st)
#pragma unroll
            for (int ti = 0; ti < TM; ++ti)
#pragma unroll
                for (int tj = 0; tj < 2; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x2f32(b8[tj][st], a8[ti][st], acc[ti][tj], 0, 0, 0);
    }
    // register r of lane (l32, lh) of acc[ti][tj] holds
    // C[32 ti + l32][wn + 32 tj + 8 (r / 4) + 4 lh + r % 4]; half h = rows 32 h ..
    const floatx4 bv = ld_v4(g.bias + 4 * lane);
    const float4 ww = *reinterpret_cast<const float4*>(lnw + 4 * lane);
    const float4 wb = *reinterpret_cast<const float4*>(lnb + 4 * lane);
#pragma unroll
    for (int h = 0; h < TM; ++h) {
        // this wave's eight rows of the half: residual segments loaded
        // before the staging barriers (rows past M read R's first row)
        floatx4 rv[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int m = m0 + 32 * h + 8 * wave + r;
            rv[r] = ld_v4(g.R + (m < g.M ? (long)m * g.ldr + 4 * lane : 0L));
        }
        __syncthreads();   // the stages are free (main loop done / previous half consumed)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<floatx4*>(smem + l32 * RL_SST + wn + 32 * tj + 8 * q + 4 * lh) =
                    floatx4{acc[h][tj][4 * q], acc[h][tj][4 * q + 1], acc[h][tj][4 * q + 2], acc[h][tj][4 * q + 3]};
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int lr = 8 * wave + r, m = m0 + 32 * h + lr;
            if (m >= g.M) break;   // uniform over the wave; later rows are past M too
            const floatx4 v = *reinterpret_cast<const floatx4*>(smem + lr * RL_SST + 4 * lane);
            const floatx4 x = (v + bv) + rv[r];
            st_g4(g.C + (long)m * g.ldc + 4 * lane, x);
            const float mu = wave_sum((x[0] + x[1]) + (x[2] + x[3])) / (float)RL_N;
            const float a = x[0] - mu, b = x[1] - mu, c = x[2] - mu, d = x[3] - mu;
            const float var = wave_sum((a * a + b * b) + (c * c + d * d)) / (float)RL_N;
            const float rs = 1.0f / sqrtf(var + 1e-5f);
            if (lane == 0) {
                mean[m] = mu;
                rstd[m] = rs;
            }
            float4 o;
            o.x = (x[0] - mu) * rs * ww.x + wb.x;
            o.y = (x[1] - mu) * rs * ww.y + wb.y;
            o.z = (x[2] - mu) * rs * ww.z + wb.z;
            o.w = (x[3] - mu) * rs * ww.w + wb.w;
            if constexpr (YB)
                *reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(Y) + (long)m * ldy + 4 * lane) =
                    bf16x4{(__bf16)o.x, (__bf16)o.y, (__bf16)o.z, (__bf16)o.w};
            else
                *reinterpret_cast<float4*>(Y + (long)m * ldy + 4 * lane) = o;
        }
    }
}

// The LayerNorm backward fused into the bf16 dX product that feeds it (the
// bf16 blocks' QKV and FFN1 dX): dy = dY W (dY rows x K bf16, W^T copy 256 x
// K bf16, k-contiguous both) never leaves the chip.  The main loop is
// gemm_resid_ln_kernel's bf16 one on 128 x 256 tiles; the epilogue stages dy
// in 32-row halves and a wave takes eight rows, one float4 per lane, in
// ln_bwd_kernel's arithmetic: dx = rs (g - mean(g) - xh mean(g xh)) + dres
// with g = dy w, xh = (x - mu) rs, written fp32 and as a bf16 copy.  The
// LayerNorm parameter gradients' per-row terms dy xh and dy are summed per
// lane over the wave's rows, then over the four waves in order, into one
// partial row of 512 floats per workgroup (part); workgroups past the device
// row count write zeros there, so the column sum over every workgroup's row
// is complete.
struct LnBwdArgs {
    const float* x; const float* mean; const float* rstd; const float* w; const float* dres;
    float* dx; __bf16* dxh; float* part;
};
template <int BMR>
__global__ __launch_bounds__(NT) void gemm_dx_lnbwd_kernel(const GemmArgs g0, const LnBwdArgs a) {
    const GemmArgs g = gemm_shape(g0);
    static_assert(BMR == 64 || BMR == 128, "64- or 128-row tiles");
    constexpr int TM = BMR / 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.x * BMR;
    if (m0 >= g.M) {   // beyond the (device) row count: a zero partial row
        for (int c = tid; c < 2 * RL_N; c += NT) a.part[(long)blockIdx.x * 2 * RL_N + c] = 0.f;
        return;
    }
    constexpr int TA = BMR * BK, TB = RL_N * BK, STAGE = TA + TB;
    constexpr int SMEM = 2 * STAGE > 32 * RL_SST ? 2 * STAGE : 32 * RL_SST;
    __shared__ __align__(16) float smem[SMEM];
    const int l32 = lane & 31, lh = lane >> 5;
    const int wn = 64 * wave;
    floatx16 acc[TM][2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const unsigned ea = (unsigned)(((long)(g.M - 1) * g.lda + g.K) * 4);
    const unsigned eb = (unsigned)(((long)(RL_N - 1) * g.ldb + g.K) * 4);
    const int32x4_t ra = buffer_rsrc(g.A, ea), rb = buffer_rsrc(g.B, eb);
    // A's 16-row chunks: chunk wave (and wave + 4 for 128-row tiles)
    const int sa = dma_src<false>(wave, lane, m0, g.lda), sa2 = dma_src<false>(wave + 4, lane, m0, g.lda);
    int sb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sb[j] = dma_src<false>(4 * wave + j, lane, 0, g.ldb);
    auto issue = [&](int tile) {
        const int k0 = tile * BK;
        const float* st = smem + (tile & 1) * STAGE;
        dma16(ra, st + wave * 256, (sa + k0) * 4);
        if (BMR == 128) dma16(ra, st + (wave + 4) * 256, (sa2 + k0) * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16(rb, st + TA + (4 * wave + j) * 256, (sb[j] + k0) * 4);
    };
    const int nk = g.K / BK;
    issue(0);
    for (int it = 0; it < nk; ++it) {
        wait_vm<0>();
        __syncthreads();
        if (it + 1 < nk) issue(it + 1);
        const float* Ab = smem + (it & 1) * STAGE;
        const float* Bb = Ab + TA;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            bf16x8 ah[TM], bh[2];
#pragma unroll
            for (int t = 0; t < TM; ++t)
                ah[t] = *reinterpret_cast<const bf16x8*>(Ab + dma_at<false>(32 * t + l32, 4 * (2 * st + lh)));
#pragma unroll
            for (int t = 0; t < 2; ++t)
                bh[t] = *reinterpret_cast<const bf16x8*>(Bb + dma_at<false>(wn + 32 * t + l32, 4 * (2 * st + lh)));
#pragma unroll
            for (int ti = 0; ti < TM; ++ti)
#pragma unroll
                for (int tj = 0; tj < 2; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh[tj], ah[ti], acc[ti][tj], 0, 0, 0);
        }
    }
    const float4 wv = *reinterpret_cast<const float4*>(a.w + 4 * lane);
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 aw = z4, ab = z4;
    const int mlast = g.M - 1;
    // a row's x, residual gradient and statistics are loaded one row ahead
    // (row indices clamped to the last row, so every load is in bounds)
    auto ld_row = [&](int m, float4& xv, float4& rv, float& mu, float& rs) {
        xv = *reinterpret_cast<const float4*>(a.x + (long)m * RL_N + 4 * lane);
        rv = a.dres ? *reinterpret_cast<const float4*>(a.dres + (long)m * RL_N + 4 * lane) : z4;
        mu = a.mean[m];
        rs = a.rstd[m];
    };
#pragma unroll
    for (int h = 0; h < TM; ++h) {
        const int mb = m0 + 32 * h + 8 * wave;
        float4 xv, rv;
        float mu, rs;
        ld_row(mb < mlast ? mb : mlast, xv, rv, mu, rs);
        __syncthreads();   // the stages are free (main loop done / previous half consumed)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<floatx4*>(smem + l32 * RL_SST + wn + 32 * tj + 8 * q + 4 * lh) =
                    floatx4{acc[h][tj][4 * q], acc[h][tj][4 * q + 1], acc[h][tj][4 * q + 2], acc[h][tj][4 * q + 3]};
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int lr = 8 * wave + r, m = mb + r;
            if (m >= g.M) break;   // uniform over the wave; later rows are past M too
            float4 xn, rn;
            float mun, rsn;
            ld_row(m < mlast ? m + 1 : mlast, xn, rn, mun, rsn);
            const float4 dd = *reinterpret_cast<const float4*>(smem + lr * RL_SST + 4 * lane);
            const float4 xh = make_float4((xv.x - mu) * rs, (xv.y - mu) * rs, (xv.z - mu) * rs, (xv.w - mu) * rs);
            const float4 gv = make_float4(dd.x * wv.x, dd.y * wv.y, dd.z * wv.z, dd.w * wv.w);
            const float s1 = (gv.x + gv.y) + (gv.z + gv.w);
            const float s2 = (gv.x * xh.x + gv.y * xh.y) + (gv.z * xh.z + gv.w * xh.w);
            aw.x += dd.x * xh.x; aw.y += dd.y * xh.y; aw.z += dd.z * xh.z; aw.w += dd.w * xh.w;
            ab.x += dd.x; ab.y += dd.y; ab.z += dd.z; ab.w += dd.w;
            const float m1 = wave_sum(s1) / (float)RL_N;
            const float m2 = wave_sum(s2) / (float)RL_N;
            float4 o;
            o.x = (gv.x - m1 - xh.x * m2) * rs;
            o.y = (gv.y - m1 - xh.y * m2) * rs;
            o.z = (gv.z - m1 - xh.z * m2) * rs;
            o.w = (gv.w - m1 - xh.w * m2) * rs;
            if (a.dres) {
                o.x += rv.x; o.y += rv.y; o.z += rv.z; o.w += rv.w;
            }
            *reinterpret_cast<float4*>(a.dx + (long)m * RL_N + 4 * lane) = o;
            if (a.dxh)
                *reinterpret_cast<bf16x4*>(a.dxh + (long)m * RL_N + 4 * lane) =
                    bf16x4{(__bf16)o.x, (__bf16)o.y, (__bf16)o.z, (__bf16)o.w};
            xv = xn; rv = rn; mu = mun; rs = rsn;
        }
    }
    // the workgroup's partial row: [sum dy xh (256) | sum dy (256)], waves in order
    __syncthreads();   // the stage is free
    float* red = smem;   // [4 waves][512]
    *reinterpret_cast<float4*>(red + wave * 2 * RL_N + 4 * lane) = aw;
    *reinterpret_cast<float4*>(red + wave * 2 * RL_N + RL_N + 4 * lane) = ab;
    __syncthreads();
    for (int c = tid; c < 2 * RL_N; c += NT)
        a.part[(long)blockIdx.x * 2 * RL_N + c] =
            ((red[c] + red[2 * RL_N + c]) + red[4 * RL_N + c]) + red[6 * RL_N + c];
}

// Grouped launch: several independent products (different shapes and
// operands, one layout and epilogue) in one grid.  Work item w belongs to
// product item_group[w]; its logical tile and K split follow from the
// product's first item, tile count and split count.
template <bool AT, bool BT, int EPI, bool PARTIAL>
__global__ __launch_bounds__(NT) void gemm_f32_dma_grouped_kernel(const GroupedGemm* __restrict__ gs,
                                                                  const int* __restrict__ item_group) {
    __shared__ __align__(16) float smem[dma_smem_floats<DMA_NS>()];
    const int gi = __builtin_amdgcn_readfirstlane(item_group[blockIdx.x]);
    const int local = (int)blockIdx.x - gs[gi].first;
    const int tiles = gs[gi].tiles;
    gemm_dma_tile<AT, BT, EPI, PARTIAL, false>(gs[gi].g, gs[gi].k_chunk, gs[gi].part_stride, local % tiles,
                                               local / tiles, gs[gi].splits, smem);
}

// Fixed-order sums of grouped split-K partials: chunk c covers 1024
// elements of product chunk_group[c]'s C (row-major M x N at ldc; partial z
// at g.C + z * part_stride, the sum goes to out).
__global__ __launch_bounds__(256) void grouped_reduce_kernel(const GroupedGemm* __restrict__ gs,
                                                             const int* __restrict__ chunk_group,
                                                             const int* __restrict__ chunk_first) {
    const int gi = chunk_group[blockIdx.x];
    const GemmArgs& g = gs[gi].g;
    float* out = gs[gi].out;
    const int splits = gs[gi].splits;
    const long ps = gs[gi].part_stride;
    const long base = (long)((int)blockIdx.x - chunk_first[gi]) * 1024;
    const long total = (long)g.M * g.N;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const long e = base + k * 256 + threadIdx.x;
        if (e >= total) break;
        const long m = e / g.N, n = e % g.N;
        const long o = m * g.ldc + n;
        float v = g.C[o];
        for (int z = 1; z < splits; ++z) v += g.C[z * ps + o];
        out[o] = v;
    }
}

// ---------------------------------------------------------------- bf16
// Mixed precision, register-staged (shapes off the DMA rules; the DMA ones
// run gemm_bf16_k16_kernel): fp32 operands from HBM are rounded to bf16
// (RNE) on the way into LDS and multiplied on v_mfma_f32_16x16x32_bf16 with
// fp32 accumulation; the epilogue is the fp32 kernel's.  Same 128x128 block,
// 4 waves x 64x64, XCD tile order; BK = 32 (one MFMA k-step).  Both operands
// sit in LDS as [row][k] bf16 (row stride 40: 16 B-aligned 128-bit fragment
// reads, conflict-free across 8 lanes); an m-contiguous operand is
// transposed in registers (4x4 blocks) before its 64-bit LDS stores.  A
// lane's fragment is 8 consecutive k of one row; A and B use the same
// (lane group, element) -> k map, so the product is independent of the
// hardware's internal k order.
constexpr int BK2 = 32, SKB2 = BK2 + 8;

// stage one operand's 128 x 32 tile: T (m-contiguous in memory) or not.
// Thread t covers: !T: row t/2, k 16*(t%2) .. +15 (four 128-bit loads);
// T: rows 4*(t/8) .. +3, k 4*(t%8) .. +3 (four 128-bit loads along m).
template <bool T>
__device__ __forceinline__ void bf_load(const gfloat* X, long ld, int lim, int r0, int k0, int kend, int tid,
                                        float4 (&v)[4]) {
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!T) {
        const int row = r0 + (tid >> 1), kq = k0 + (tid & 1) * 16;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = (row < lim && kq + 4 * j < kend) ? ld_g4(X + (long)row * ld + kq + 4 * j) : z4;
    } else {
        const int mq = r0 + (tid >> 3) * 4, kq = k0 + (tid & 7) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = (mq < lim && kq + j < kend) ? ld_g4(X + (long)(kq + j) * ld + mq) : z4;
    }
}

template <bool T>
__device__ __forceinline__ void bf_store(__bf16* S, int tid, const float4 (&v)[4]) {
    if (!T) {
        const int row = tid >> 1, kq = (tid & 1) * 16;
        bf16x4* d = reinterpret_cast<bf16x4*>(S + row * SKB2 + kq);
#pragma unroll
        for (int j = 0; j < 4; ++j) d[j] = to_bf16x4(v[j].x, v[j].y, v[j].z, v[j].w);
    } else {
        const int mq = (tid >> 3) * 4, kq = (tid & 7) * 4;
        *reinterpret_cast<bf16x4*>(S + (mq + 0) * SKB2 + kq) = to_bf16x4(v[0].x, v[1].x, v[2].x, v[3].x);
        *reinterpret_cast<bf16x4*>(S + (mq + 1) * SKB2 + kq) = to_bf16x4(v[0].y, v[1].y, v[2].y, v[3].y);
        *reinterpret_cast<bf16x4*>(S + (mq + 2) * SKB2 + kq) = to_bf16x4(v[0].z, v[1].z, v[2].z, v[3].z);
        *reinterpret_cast<bf16x4*>(S + (mq + 3) * SKB2 + kq) = to_bf16x4(v[0].w, v[1].w, v[2].w, v[3].w);
    }
}

template <bool AT, bool BT, int EPI, bool PARTIAL>
__global__ __launch_bounds__(NT) void gemm_bf16_kernel(const GemmArgs g0, int k_chunk0, long part_stride) {
    const GemmArgs g = gemm_shape(g0);
    // a device reduction count splits its own K evenly over the launch's splits
    const int k_chunk = g0.Kdev ? (((g.K + (int)gridDim.z - 1) / (int)gridDim.z + BK2 - 1) / BK2) * BK2 : k_chunk0;
    constexpr int SMEM = 2 * (BM + BN) * SKB2 / 2;   // floats
    static_assert(SMEM >= STAGE_FLOATS, "epilogue stage does not fit the operand stages");
    __shared__ __align__(16) float smem[SMEM];
    __bf16 (*As)[BM * SKB2] = reinterpret_cast<__bf16 (*)[BM * SKB2]>(smem);
    __bf16 (*Bs)[BN * SKB2] = reinterpret_cast<__bf16 (*)[BN * SKB2]>(smem + BM * SKB2);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tn = (g.N + BN - 1) / BN;
    int tmi, tni;
    if (!tile_of_range(g, tn, tmi, tni, blockIdx.x)) return;   // beyond the (device) tile count
    const int m0 = tmi * BM, n0 = tni * BN;
    const int kbeg = blockIdx.z * k_chunk;
    const int kend = min(g.K, kbeg + k_chunk);
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int li = lane & 15, lq = lane >> 4;
    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    const gfloat* __restrict__ Ag = (const gfloat*)(g.A);
    const gfloat* __restrict__ Bg = (const gfloat*)(g.B);
    float4 va[4], vb[4];
    if (kbeg < kend) {
        bf_load<AT>(Ag, g.lda, g.M, m0, kbeg, kend, tid, va);
        bf_load<BT>(Bg, g.ldb, g.N, n0, kbeg, kend, tid, vb);
        bf_store<AT>(As[0], tid, va);
        bf_store<BT>(Bs[0], tid, vb);
        __syncthreads();
        int buf = 0;
        for (int k0 = kbeg; k0 < kend; k0 += BK2) {
            const bool more = k0 + BK2 < kend;
            if (more) {
                bf_load<AT>(Ag, g.lda, g.M, m0, k0 + BK2, kend, tid, va);
                bf_load<BT>(Bg, g.ldb, g.N, n0, k0 + BK2, kend, tid, vb);
            }
            bf16x8 af[4], bfr[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                af[t] = *reinterpret_cast<const bf16x8*>(&As[buf][(wm + t * 16 + li) * SKB2 + 8 * lq]);
                bfr[t] = *reinterpret_cast<const bf16x8*>(&Bs[buf][(wn + t * 16 + li) * SKB2 + 8 * lq]);
            }
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int tj = 0; tj < 4; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[tj], af[ti], acc[ti][tj], 0, 0, 0);
            if (more) {
                bf_store<AT>(As[buf ^ 1], tid, va);
                bf_store<BT>(Bs[buf ^ 1], tid, vb);
            }
            __syncthreads();
            buf ^= 1;
        }
    }
    gemm_epilogue<EPI, PARTIAL>(g, acc, m0, n0, wm, wn, li, lq, part_stride, smem, blockIdx.z);
}

// ---------------------------------------------------------------- bf16, LDS DMA
// bf16 products on the fp32 DMA pipeline (16 k per stage, operands rounded
// as they leave LDS; bias sums of the fp32 tiles as in the fp32 kernel).
// Three stages: deeper pipelines measured no faster (the loop is bound by
// the operand fetches, not their latency).
constexpr int BF_NS = 3;
template <bool AT, bool BT, int EPI, bool PARTIAL, bool DB>
__global__ __launch_bounds__(NT) void gemm_bf16_k16_kernel(const GemmArgs g0, int k_chunk0, long part_stride) {
    __shared__ __align__(16) float smem[dma_smem_floats<BF_NS>()];
    gemm_dma_tile<AT, BT, EPI, PARTIAL, DB, true, BF_NS>(g0, k_chunk0, part_stride, blockIdx.x, blockIdx.z,
                                                         gridDim.z, smem);
}

// ---------------------------------------------------------------- bf16 activations
// Products whose operands are stored in bf16 (the mixed-precision variant's
// activations and bf16 copies of the weights), fp32 accumulation.
//
// gemm_bs32_kernel: C = epi(A B^T), A (M, K) and B (N, K) bf16, both
// k-contiguous, shapes in float units: the fp32 kernel's LDS-DMA stages and
// layouts with the bytes reinterpreted (a 16-float stage row is 32 bf16 k,
// a 4-float group 8 of them), multiplied on v_mfma_f32_32x32x16_bf16 (1.7x
// the rate of the 16 x 16 form on this GPU; measured 1-4% faster than a
// 16 x 16 x 32 version of this kernel, whose loop waits on its operand
// fetches rather than on the matrix pipe).  A wave's 64 x 64 tile is 2 x 2
// MFMA tiles of 32 x 32, two 16-k steps per 32-k stage.  Lane (l32 = lane % 32, lh = lane / 32) supplies row
// l32 of its 32-row slice and k = 8 lh .. 8 lh + 7 of the step — the 16 B
// group 2 s + lh of the stage row — for both A and B.  With B as the first
// operand, accumulator register r of lane (l32, lh) holds
// C[wm + 32 ti + l32][wn + 32 tj + 8 (r / 4) + 4 lh + r % 4]: four runs of
// four consecutive columns of one row, staged through LDS as the 16 x 16
// kernels' epilogue does (half h = rows wm + 32 h .. + 31 of both wave rows).
template <int EPI, bool OB, int NS>
__global__ __launch_bounds__(NT) void gemm_bs32_kernel(const GemmArgs g0) {
    const GemmArgs g = gemm_shape(g0);
    constexpr int TILE = BM * BK;   // floats per operand stage (BM == BN)
    constexpr int SMEM = NS * 2 * TILE > STAGE_FLOATS ? NS * 2 * TILE : STAGE_FLOATS;
    __shared__ __align__(16) float smem[SMEM];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tn = (g.N + BN - 1) / BN;
    int tmi, tni;
    if (!tile_of_range(g, tn, tmi, tni, blockIdx.x)) return;
    const int m0 = tmi * BM, n0 = tni * BN;
    const int nk = (g.K + BK - 1) / BK;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int l32 = lane & 31, lh = lane >> 5;
    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const unsigned ea = (unsigned)((long)(g.M - 1) * g.lda + g.K) * 4u;
    const unsigned eb = (unsigned)((long)(g.N - 1) * g.ldb + g.K) * 4u;
    const int32x4_t ra = buffer_rsrc(g.A, ea), rb = buffer_rsrc(g.B, eb);
    const int sa0 = dma_src<false>(2 * wave, lane, m0, g.lda), sa1 = dma_src<false>(2 * wave + 1, lane, m0, g.lda);
    const int sb0 = dma_src<false>(2 * wave, lane, n0, g.ldb), sb1 = dma_src<false>(2 * wave + 1, lane, n0, g.ldb);
    // multiply epilogue on bf16 (the GELU derivative): the first half's R
    // segments load before the main loop, the second half's after it, so the
    // epilogue does not wait on them
    constexpr bool RPF = EPI == EPI_MUL && OB;
    const uintptr_t al8 = (uintptr_t)g.C | (uintptr_t)g.C2 | (uintptr_t)g.R | (uintptr_t)((g.ldc | g.ldc2 | g.ldr) * 2);
    const uintptr_t al = (uintptr_t)g.C | (uintptr_t)g.C2 | (uintptr_t)g.R | (uintptr_t)g.bias |
                         (uintptr_t)((g.ldc | g.ldc2 | g.ldr) * 4);
    const bool vo8 = (al & 15) == 0 && (al8 & 15) == 0;
    bf16x8 rpf[2][4];
    auto load_r = [&](int h) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int it = tid + j * NT, lr = it / (BN / 8), c = (it % (BN / 8)) * 8;
            const int m = m0 + (lr >> 5) * 64 + 32 * h + (lr & 31), n = n0 + c;
            if (m < g.M && n + 7 < g.N)
                rpf[h][j] = *reinterpret_cast<const bf16x8*>(bfp(g.R) + (long)m * g.ldr + n);
        }
    };
    if (RPF && vo8) load_r(0);
#define PT_ISSUE32(tile)                                                                \
    {                                                                                   \
        const int k0_ = (tile) * BK;                                                    \
        const float* st_ = smem + ((tile) % NS) * 2 * TILE;                             \
        dma16(ra, st_ + (2 * wave) * 256, (sa0 + k0_) * 4);                             \
        dma16(ra, st_ + (2 * wave + 1) * 256, (sa1 + k0_) * 4);                         \
        dma16(rb, st_ + TILE + (2 * wave) * 256, (sb0 + k0_) * 4);                      \
        dma16(rb, st_ + TILE + (2 * wave + 1) * 256, (sb1 + k0_) * 4);                  \
    }
    if (nk > 0) {
#pragma unroll
        for (int t = 0; t < NS - 1; ++t)
            if (t < nk) PT_ISSUE32(t)
        for (int it = 0; it < nk; ++it) {
            wait_stages<NS>(min(NS - 2, nk - 1 - it));
            __syncthreads();   // every wave's loads of stage it are in LDS; stage it - 1 is consumed
            const int kv = g.K - it * BK;   // floats of this stage inside K
            if (kv < BK) {
                float* st = smem + (it % NS) * 2 * TILE;
                for (int idx = tid; idx < BM * BK; idx += NT) {
                    const int r = idx / BK, k = idx % BK;
                    if (k >= kv) {
                        st[dma_at<false>(r, k)] = 0.f;
                        st[TILE + dma_at<false>(r, k)] = 0.f;
                    }
                }
                __syncthreads();
            }
            if (it + NS - 1 < nk) PT_ISSUE32(it + NS - 1)
            const float* Ab = smem + (it % NS) * 2 * TILE;
            const float* Bb = Ab + TILE;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                bf16x8 ah[2], bh[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    ah[t] = *reinterpret_cast<const bf16x8*>(Ab + dma_at<false>(wm + 32 * t + l32, 4 * (2 * st + lh)));
                    bh[t] = *reinterpret_cast<const bf16x8*>(Bb + dma_at<false>(wn + 32 * t + l32, 4 * (2 * st + lh)));
                }
#pragma unroll
                for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                    for (int tj = 0; tj < 2; ++tj)
                        acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh[tj], ah[ti], acc[ti][tj], 0, 0, 0);
            }
        }
    }
#undef PT_ISSUE32
    if constexpr (RPF) {
        if (vo8) {
            load_r(1);
            // 16 B bf16 stores of C = acc * R with the prefetched R (same
            // staging and arithmetic as epilogue_staged32's EPI_MUL path)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                __syncthreads();
#pragma unroll
                for (int tj = 0; tj < 2; ++tj)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *reinterpret_cast<floatx4*>(smem + ((wm >> 6) * 32 + l32) * SST + wn + 32 * tj + 8 * q +
                                                    4 * lh) =
                            floatx4{acc[h][tj][4 * q], acc[h][tj][4 * q + 1], acc[h][tj][4 * q + 2],
                                    acc[h][tj][4 * q + 3]};
                __syncthreads();
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int it = tid + j * NT, lr = it / (BN / 8), c = (it % (BN / 8)) * 8;
                    const int m = m0 + (lr >> 5) * 64 + 32 * h + (lr & 31), n = n0 + c;
                    if (m >= g.M || n >= g.N) continue;
                    const floatx4 v0 = *reinterpret_cast<const floatx4*>(smem + lr * SST + c);
                    const floatx4 v1 = *reinterpret_cast<const floatx4*>(smem + lr * SST + c + 4);
                    if (n + 7 < g.N) {
                        const bf16x8 r = rpf[h][j];
                        st_b8(g.C, (long)m * g.ldc + n,
                              v0 * floatx4{(float)r[0], (float)r[1], (float)r[2], (float)r[3]},
                              v1 * floatx4{(float)r[4], (float)r[5], (float)r[6], (float)r[7]});
                    } else {
                        for (int e = 0; e < 4 && n + e < g.N; ++e) epi_store<EPI, OB>(g, m, n + e, v0[e]);
                        for (int e = 0; e < 4 && n + 4 + e < g.N; ++e) epi_store<EPI, OB>(g, m, n + 4 + e, v1[e]);
                    }
                }
            }
            return;
        }
    }
    // 16 B bf16 stores: bf16 rows of a multiple of 8 elements (R of EPI_MUL is bf16 too)
    epilogue_staged32<EPI, OB>(g, acc, m0, n0, wm, wn, l32, lh, smem, (al & 15) == 0, vo8);
}

// gemm_bs_dw_kernel: weight gradients dW (M, N) = sum_k A[k][m] B[k][n] with
// A = dY (K rows, ld lda) and B = X (K rows, ld ldb) in bf16, K = the rows
// (split across grid.z in chunks of k_chunk rows, multiples of BKW).  Both
// operands are m- (n-) contiguous, so a lane's MFMA fragment (8 consecutive
// k of one column) is strided in memory.  Each thread stages one 8 x 8 block
// per stage: 8 rows of one 16 B column chunk (16 lanes cover a 256 B row
// segment), transposed in registers (two 16-bit halves per dword), then
// written as 8 rows of 16 B into a [column][k] LDS tile; fragment reads are
// then single 128-bit reads.  LDS tile: row r (a column of the operand),
// 16 B group q at r * 64 + 8 * (q ^ f(r)), f(r) = (r ^ (r >> 3)) & 7: the
// 8 lanes of a fragment read (rows r0..r0+7, one group) and of a staging
// write (rows 8c + i for 8 consecutive c) land on 8 distinct groups.
// Register double buffering: the global loads of stage it + 1 are in flight
// while stage it is multiplied.  DB: bias sums sum_k A[k][m] from the staged
// registers (fixed order: rows within a block, stages, then the 8 blocks).
constexpr int BKW = 64;
__device__ __forceinline__ int tw_at(int r, int q) { return r * BKW + 8 * (q ^ ((r ^ (r >> 3)) & 7)); }
typedef unsigned uintx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) uintx4 guintx4;

template <bool DB, bool PARTIAL>
__global__ __launch_bounds__(NT) void gemm_bs_dw_kernel(const GemmArgs g0, int k_chunk0, long part_stride) {
    const GemmArgs g = gemm_shape(g0);
    const int gz = gridDim.z, bz = blockIdx.z;
    const int k_chunk = g0.Kdev ? (((g.K + gz - 1) / gz + BKW - 1) / BKW) * BKW : k_chunk0;
    __shared__ __align__(16) __bf16 sm[2][2][BM * BKW];   // [buffer][operand][row * 64 + k]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tn = (g.N + BN - 1) / BN;
    int tmi, tni;
    if (!tile_of_range(g, tn, tmi, tni, blockIdx.x)) return;
    const int m0 = tmi * BM, n0 = tni * BN;
    const int kbeg = bz * k_chunk;
    const int kend = min(g.K, kbeg + k_chunk);
    const int nk = kend > kbeg ? (kend - kbeg + BKW - 1) / BKW : 0;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int li = lane & 15, lq = lane >> 4;
    // staging role: operand op (0: A, 1: B), 8-column chunk cb, 8-row block kb
    const int op = tid >> 7, cb = tid & 15, kb = (tid >> 4) & 7;
    const __bf16* src = bfp(op == 0 ? g.A : g.B);
    const long ld = op == 0 ? g.lda : g.ldb;
    const int c0 = (op == 0 ? m0 : n0) + 8 * cb;
    const bool cvalid = c0 < (op == 0 ? g.M : g.N);   // M, N multiples of 8 (host)
    const bool db_blk = DB && tni == 0;               // uniform over the block
    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float dbs[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dbs[i] = 0.f;
    unsigned w[8][4];
    auto load = [&](int it) {
        const int kr = kbeg + it * BKW + 8 * kb;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uintx4 v = uintx4{0u, 0u, 0u, 0u};
            if (cvalid && kr + j < kend) v = *(const guintx4*)(src + (long)(kr + j) * ld + c0);
            w[j][0] = v[0]; w[j][1] = v[1]; w[j][2] = v[2]; w[j][3] = v[3];
        }
    };
    auto store = [&](int buf) {
        __bf16* S = &sm[buf][op][0];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 lo, hi;   // columns 2q (low halves) and 2q + 1 (high halves), rows 0..7
            lo.x = (w[0][q] & 0xffffu) | (w[1][q] << 16);
            lo.y = (w[2][q] & 0xffffu) | (w[3][q] << 16);
            lo.z = (w[4][q] & 0xffffu) | (w[5][q] << 16);
            lo.w = (w[6][q] & 0xffffu) | (w[7][q] << 16);
            hi.x = (w[0][q] >> 16) | (w[1][q] & 0xffff0000u);
            hi.y = (w[2][q] >> 16) | (w[3][q] & 0xffff0000u);
            hi.z = (w[4][q] >> 16) | (w[5][q] & 0xffff0000u);
            hi.w = (w[6][q] >> 16) | (w[7][q] & 0xffff0000u);
            *reinterpret_cast<uint4*>(S + tw_at(8 * cb + 2 * q, kb)) = lo;
            *reinterpret_cast<uint4*>(S + tw_at(8 * cb + 2 * q + 1, kb)) = hi;
            if (db_blk && op == 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    dbs[2 * q] += __uint_as_float(w[j][q] << 16);
                    dbs[2 * q + 1] += __uint_as_float(w[j][q] & 0xffff0000u);
                }
            }
        }
    };
    if (nk > 0) {
        load(0);
        store(0);
        __syncthreads();
        for (int it = 0; it < nk; ++it) {
            if (it + 1 < nk) load(it + 1);
            const __bf16* As = &sm[it & 1][0][0];
            const __bf16* Bs = &sm[it & 1][1][0];
#pragma unroll
            for (int kk = 0; kk < BKW / 32; ++kk) {
                bf16x8 ah[4], bh[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    ah[t] = *reinterpret_cast<const bf16x8*>(As + tw_at(wm + t * 16 + li, 4 * kk + lq));
                    bh[t] = *reinterpret_cast<const bf16x8*>(Bs + tw_at(wn + t * 16 + li, 4 * kk + lq));
                }
#pragma unroll
                for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                    for (int tj = 0; tj < 4; ++tj)
                        acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[tj], ah[ti], acc[ti][tj], 0, 0, 0);
            }
            if (it + 1 < nk) store((it + 1) & 1);
            __syncthreads();
        }
    }
    if (db_blk) {
        float* red = reinterpret_cast<float*>(&sm[0][0][0]);   // [8][128]
        if (op == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) red[kb * BM + 8 * cb + i] = dbs[i];
        }
        __syncthreads();
        if (tid < BM) {
            float v = 0.f;
#pragma unroll
            for (int b = 0; b < 8; ++b) v += red[b * BM + tid];
            const int m = m0 + tid;
            if (m < g.M) {
                if (PARTIAL) g.C[(long)gz * part_stride + (long)bz * g.M + m] = v;
                else g.dbias[m] = v;
            }
        }
    }
    gemm_epilogue<EPI_STORE, PARTIAL>(g, acc, m0, n0, wm, wn, li, lq, part_stride, nullptr, bz);
}

// sum_k bp[k * M] for k < splits in order: loads issued 16 at a time ahead of
// the adds (a bias partial of every split would otherwise cost one memory
// round trip each)
__device__ __forceinline__ float sum_split_column(const float* bp, int splits, int M) {
    float s = 0.f;
    int k = 0;
    for (; k + 16 <= splits; k += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = bp[(long)(k + j) * M];
#pragma unroll
        for (int j = 0; j < 16; ++j) s += v[j];
    }
    for (; k < splits; ++k) s += bp[(long)k * M];
    return s;
}

// out[m][n] (=|+=) sum_s part[s][m][n], fixed order over s
// and, when db is set, db[m] = sum_s part[splits*part_stride + s*M + m]
// V4: a thread sums 4 consecutive columns (N, ldc multiples of 4, C 16 B aligned)
// The bf16 weight gradient on 256 x 256 tiles: dW (M x N) = dY^T X over
// the rows K, A = dY (K x M) and B = X (K x N) bf16, both m-contiguous.  A
// 128 x 128 tile moves 32 KB through LDS per 64-row stage for 2.1 MFLOP and
// is bound by that operand delivery; a 256 x 256 tile moves 64 KB for 8.4
// MFLOP.  512 threads: each stages 8 rows x 8 columns of one operand through
// registers, transposed into the [column][k] LDS layout of gemm_bs_dw_kernel
// (two stages, 128 KB); eight waves of 128 x 64, each 4 x 2 tiles of
// v_mfma_f32_32x32x16_bf16 with the B fragment first (register r of lane
// (l32, lh) of acc[ti][tj] holds C[wm + 32 ti + l32][wn + 32 tj + 8 (r / 4)
// + 4 lh + r % 4]), stored straight from the accumulators.  M and N are
// multiples of 256 (host checked).
template <bool DB, bool PARTIAL>
__global__ __launch_bounds__(512) void gemm_bs_dw256_kernel(const GemmArgs g0, int k_chunk0, long part_stride) {
    constexpr int T = 256, NT2 = 512;
    const GemmArgs g = gemm_shape(g0);
    const int gz = gridDim.z, bz = blockIdx.z;
    const int k_chunk = g0.Kdev ? (((g.K + gz - 1) / gz + BKW - 1) / BKW) * BKW : k_chunk0;
    extern __shared__ __align__(16) float smw[];
    __bf16* const sm = reinterpret_cast<__bf16*>(smw);   // [buffer][operand][T * BKW]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tn = g.N / T;
    const int tmi = blockIdx.x / tn, tni = blockIdx.x % tn;
    const int m0 = tmi * T, n0 = tni * T;
    const int kbeg = bz * k_chunk;
    const int kend = min(g.K, kbeg + k_chunk);
    const int nk = kend > kbeg ? (kend - kbeg + BKW - 1) / BKW : 0;
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
    const int l32 = lane & 31, lh = lane >> 5;
    // staging role: operand op (0: A, 1: B), 8-column chunk cb (32), 8-row block kb (8)
    const int op = tid >> 8, cb = tid & 31, kb = (tid >> 5) & 7;
    const __bf16* src = bfp(op == 0 ? g.A : g.B);
    const long ld = op == 0 ? g.lda : g.ldb;
    const int c0 = (op == 0 ? m0 : n0) + 8 * cb;
    const bool db_blk = DB && tni == 0;               // uniform over the block
    floatx16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    float dbs[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dbs[i] = 0.f;
    unsigned w[8][4];
    auto load = [&](int it) {
        const int kr = kbeg + it * BKW + 8 * kb;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uintx4 v = uintx4{0u, 0u, 0u, 0u};
            if (kr + j < kend) v = *(const guintx4*)(src + (long)(kr + j) * ld + c0);
            w[j][0] = v[0]; w[j][1] = v[1]; w[j][2] = v[2]; w[j][3] = v[3];
        }
    };
    auto store = [&](int buf) {
        __bf16* S = sm + (buf * 2 + op) * (T * BKW);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 lo, hi;   // columns 2q (low halves) and 2q + 1 (high halves), rows 0..7
            lo.x = (w[0][q] & 0xffffu) | (w[1][q] << 16);
            lo.y = (w[2][q] & 0xffffu) | (w[3][q] << 16);
            lo.z = (w[4][q] & 0xffffu) | (w[5][q] << 16);
            lo.w = (w[6][q] & 0xffffu) | (w[7][q] << 16);
            hi.x = (w[0][q] >> 16) | (w[1][q] & 0xffff0000u);
            hi.y = (w[2][q] >> 16) | (w[3][q] & 0xffff0000u);
            hi.z = (w[4][q] >> 16) | (w[5][q] & 0xffff0000u);
            hi.w = (w[6][q] >> 16) | (w[7][q] & 0xffff0000u);
            *reinterpret_cast<uint4*>(S + tw_at(8 * cb + 2 * q, kb)) = lo;
            *reinterpret_cast<uint4*>(S + tw_at(8 * cb + 2 * q + 1, kb)) = hi;
            if (db_blk && op == 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    dbs[2 * q] += __uint_as_float(w[j][q] << 16);
                    dbs[2 * q + 1] += __uint_as_float(w[j][q] & 0xffff0000u);
                }
            }
        }
    };
    if (nk > 0) {
        load(0);
        store(0);
        __syncthreads();
        for (int it = 0; it < nk; ++it) {
            if (it + 1 < nk) load(it + 1);
            const __bf16* As = sm + ((it & 1) * 2) * (T * BKW);
            const __bf16* Bs = As + T * BKW;
#pragma unroll
            for (int st = 0; st < BKW / 16; ++st) {
                bf16x8 ah[4], bh[2];
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    ah[t] = *reinterpret_cast<const bf16x8*>(As + tw_at(wm + 32 * t + l32, 2 * st + lh));
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    bh[t] = *reinterpret_cast<const bf16x8*>(Bs + tw_at(wn + 32 * t + l32, 2 * st + lh));
#pragma unroll
                for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                    for (int tj = 0; tj < 2; ++tj)
                        acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh[tj], ah[ti], acc[ti][tj], 0, 0, 0);
            }
            if (it + 1 < nk) store((it + 1) & 1);
            __syncthreads();
        }
    }
    if (db_blk) {
        float* red = smw;   // [8][T] (the stages are free after the last barrier)
        if (op == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) red[kb * T + 8 * cb + i] = dbs[i];
        }
        __syncthreads();
        if (tid < T) {
            float v = 0.f;
#pragma unroll
            for (int b = 0; b < 8; ++b) v += red[b * T + tid];
            const int m = m0 + tid;
            if (PARTIAL) g.C[(long)gz * part_stride + (long)bz * g.M + m] = v;
            else g.dbias[m] = v;
        }
    }
    float* C = PARTIAL ? g.C + (long)bz * part_stride : g.C;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
        const int m = m0 + wm + 32 * ti + l32;
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn + 32 * tj + 8 * q + 4 * lh;
                st_g4(C + (long)m * g.ldc + n, floatx4{acc[ti][tj][4 * q], acc[ti][tj][4 * q + 1],
                                                       acc[ti][tj][4 * q + 2], acc[ti][tj][4 * q + 3]});
            }
    }
}

// sdev (optional): the number of partials to sum, written on the device by
// the product (at most splits, which places the bias partials)
template <bool ACCUM, bool V4>
__global__ void splitk_reduce_kernel(float* C, long ldc, const float* part, long part_stride,
                                     int splits, int M, int N, float* db, const int* sdev) {
    constexpr int W = V4 ? 4 : 1;
    const long nq = N / W;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int ns = sdev ? *sdev : splits;
    if (i >= (long)M * nq) {
        const long m = i - (long)M * nq;
        if (db != nullptr && m < M) db[m] = sum_split_column(part + (long)splits * part_stride + m, ns, M);
        return;
    }
    const int m = (int)(i / nq), n = (int)(i % nq) * W;
    const long o = (long)m * ldc + n;
    if (V4) {
        floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (int k = 0; k < ns; ++k) s += ld_v4(part + (long)k * part_stride + o);
        st_g4(C + o, ACCUM ? ld_v4(C + o) + s : s);
    } else {
        float s = 0.f;
#pragma unroll 8
        for (int k = 0; k < ns; ++k) s += part[(long)k * part_stride + o];
        if (ACCUM) C[o] += s; else C[o] = s;
    }
}

// The same sum for many splits (N, ldc multiples of 4, C 16 B aligned),
// parallel over split groups: block b covers 256 / G float4 outputs, group g
// of its threads sums splits [g S / G, (g + 1) S / G) in order, and the G
// group sums are added in group order through LDS -- a fixed order, so the
// result does not depend on scheduling.  Blocks past the outputs sum the
// bias partials (db) as splitk_reduce_kernel does.
template <bool ACCUM, int G>
__global__ __launch_bounds__(256) void splitk_reduce_grp_kernel(float* C, long ldc, const float* part,
                                                                long part_stride, int splits, int M, int N,
                                                                float* db, int out_blocks, const int* sdev) {
    constexpr int CPB = 256 / G;
    __shared__ floatx4 sh[G][CPB];
    const int t = threadIdx.x;
    const int ns = sdev ? *sdev : splits;
    if ((int)blockIdx.x >= out_blocks) {
        const int m = ((int)blockIdx.x - out_blocks) * 256 + t;
        if (db != nullptr && m < M) db[m] = sum_split_column(part + (long)splits * part_stride + m, ns, M);
        return;
    }
    const int nq = N / 4;
    const int g = t / CPB, c = t % CPB;
    const long i = (long)blockIdx.x * CPB + c;
    const bool live = i < (long)M * nq;
    const int m = live ? (int)(i / nq) : 0, n = live ? (int)(i % nq) * 4 : 0;
    const long o = (long)m * ldc + n;
    floatx4 sum = floatx4{0.f, 0.f, 0.f, 0.f};
    if (live) {
        const int zb = (int)(((long)ns * g) / G), ze = (int)(((long)ns * (g + 1)) / G);
#pragma unroll 4
        for (int z = zb; z < ze; ++z) sum += ld_v4(part + (long)z * part_stride + o);
    }
    sh[g][c] = sum;
    __syncthreads();
    if (g == 0 && live) {
        floatx4 v = sh[0][c];
#pragma unroll
        for (int k = 1; k < G; ++k) v += sh[k][c];
        st_g4(C + o, ACCUM ? ld_v4(C + o) + v : v);
    }
}

// Split-K for a product whose epilogue needs the whole sum (bias, GELU,
// residual, multiply): C = epi(sum_s part[s]) in split order, one thread per
// four columns (v4: C, C2, R, bias and leading dimensions 16 B aligned and
// N a multiple of 4) or per element.
template <int EPI, bool V4>
__global__ void splitk_epi_reduce_kernel(GemmArgs g, const float* __restrict__ part, long part_stride,
                                         int splits) {
    constexpr int W = V4 ? 4 : 1;
    const long nq = g.N / W;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)g.M * nq) return;
    const int m = (int)(i / nq), n = (int)(i % nq) * W;
    const long o = (long)m * g.ldc + n;
    if (V4) {
        floatx4 sum = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (int z = 0; z < splits; ++z) sum += ld_v4(part + (long)z * part_stride + o);
        epi_store4<EPI>(g, m, n, sum);
    } else {
        float sum = 0.f;
#pragma unroll 8
        for (int z = 0; z < splits; ++z) sum += part[(long)z * part_stride + o];
        epi_store<EPI>(g, m, n, sum);
    }
}

template <bool V4>
int launch_splitk_epi_reduce(const GemmArgs& g, const float* part, long part_stride, int splits, hipStream_t s) {
    const dim3 gr(pt_cdiv((long)g.M * (g.N / (V4 ? 4 : 1)), 256));
    switch (g.epi) {
        case EPI_BIAS: hipLaunchKernelGGL((splitk_epi_reduce_kernel<EPI_BIAS, V4>), gr, dim3(256), 0, s, g, part, part_stride, splits); break;
        case EPI_BIAS_GELU: hipLaunchKernelGGL((splitk_epi_reduce_kernel<EPI_BIAS_GELU, V4>), gr, dim3(256), 0, s, g, part, part_stride, splits); break;
        case EPI_BIAS_RESID: hipLaunchKernelGGL((splitk_epi_reduce_kernel<EPI_BIAS_RESID, V4>), gr, dim3(256), 0, s, g, part, part_stride, splits); break;
        case EPI_GELU_BWD: hipLaunchKernelGGL((splitk_epi_reduce_kernel<EPI_GELU_BWD, V4>), gr, dim3(256), 0, s, g, part, part_stride, splits); break;
        case EPI_BIAS_GELU_D: hipLaunchKernelGGL((splitk_epi_reduce_kernel<EPI_BIAS_GELU_D, V4>), gr, dim3(256), 0, s, g, part, part_stride, splits); break;
        case EPI_MUL: hipLaunchKernelGGL((splitk_epi_reduce_kernel<EPI_MUL, V4>), gr, dim3(256), 0, s, g, part, part_stride, splits); break;
        case EPI_AXPBY: hipLaunchKernelGGL((splitk_epi_reduce_kernel<EPI_AXPBY, V4>), gr, dim3(256), 0, s, g, part, part_stride, splits); break;
        default: PT_REQUIRE(false, "gemm: split-K epilogue %d not supported", g.epi);
    }
    return PTCG_OK;
}

// split-K partial sums into C (and the bias partials into db): the grouped
// form for many splits with 128-bit columns, else one thread per output
template <bool ACCUM>
void launch_splitk_reduce(float* C, long ldc, const float* part, long part_stride, int splits, int M, int N,
                          float* db, bool v4, hipStream_t s, const int* sdev = nullptr) {
    const int G = !v4 ? 1 : splits >= 64 ? 8 : splits >= 24 ? 4 : splits >= 12 ? 2 : 1;
    if (G > 1) {
        const long outs = (long)M * (N / 4);
        const int ob = pt_cdiv(outs, 256 / G), dbb = db ? pt_cdiv(M, 256) : 0;
        const dim3 gr(ob + dbb);
        if (G == 8)
            hipLaunchKernelGGL((splitk_reduce_grp_kernel<ACCUM, 8>), gr, dim3(256), 0, s, C, ldc, part, part_stride,
                               splits, M, N, db, ob, sdev);
        else if (G == 4)
            hipLaunchKernelGGL((splitk_reduce_grp_kernel<ACCUM, 4>), gr, dim3(256), 0, s, C, ldc, part, part_stride,
                               splits, M, N, db, ob, sdev);
        else
            hipLaunchKernelGGL((splitk_reduce_grp_kernel<ACCUM, 2>), gr, dim3(256), 0, s, C, ldc, part, part_stride,
                               splits, M, N, db, ob, sdev);
        return;
    }
    const long tot = (long)M * (v4 ? N / 4 : N) + (db ? M : 0);
    const dim3 gr(pt_cdiv(tot, 256));
    if (v4)
        hipLaunchKernelGGL((splitk_reduce_kernel<ACCUM, true>), gr, dim3(256), 0, s, C, ldc, part, part_stride,
                           splits, M, N, db, sdev);
    else
        hipLaunchKernelGGL((splitk_reduce_kernel<ACCUM, false>), gr, dim3(256), 0, s, C, ldc, part, part_stride,
                           splits, M, N, db, sdev);
}

// Tail tiles of a balanced launch: C[tile] = epi(sum_s part[s][tile]), fixed order over s.
template <int EPI>
__global__ void tail_reduce_kernel(GemmArgs g, const float* __restrict__ part, int splits) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)g.ntiles * BM * BN) return;
    const int t = (int)(i / (BM * BN)), e = (int)(i % (BM * BN));
    const int tn = (g.N + BN - 1) / BN;
    const int lt = g.tile0 + t;
    const int m = (lt / tn) * BM + e / BN, n = (lt % tn) * BN + e % BN;
    if (m >= g.M || n >= g.N) return;
    float v = 0.f;
    for (int z = 0; z < splits; ++z) v += part[((long)z * g.ntiles + t) * (BM * BN) + e];
    epi_store<EPI>(g, m, n, v);
}

// Deterministic column sums in two levels.  Level 1: block (64 columns x 4
// row groups) sums one slice of rows; level 2: the same shape sums the
// slice partials.  Every add happens in a fixed order.
// column sums of X (M x N) in one launch: row group g (16 of them) of a
// column sums rows g, g + 16, ... in four interleaved accumulators, then the
// sixteen group sums add in order; columns below split go to out, the rest
// to out_hi
__global__ __launch_bounds__(1024) void colsum_one_kernel(const float* __restrict__ X, long ldx, int M, int N,
                                                          float* __restrict__ out, int split,
                                                          float* __restrict__ out_hi) {
    __shared__ float sh[16][64];
    const int c = blockIdx.x * 64 + (threadIdx.x & 63);
    const int rg = threadIdx.x >> 6;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    if (c < N) {
        int r = rg;
        for (; r + 48 < M; r += 64) {
            s0 += X[(long)r * ldx + c];
            s1 += X[(long)(r + 16) * ldx + c];
            s2 += X[(long)(r + 32) * ldx + c];
            s3 += X[(long)(r + 48) * ldx + c];
        }
        for (; r < M; r += 16) s0 += X[(long)r * ldx + c];
    }
    sh[rg][threadIdx.x & 63] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (rg == 0 && c < N) {
        float v = 0.f;
#pragma unroll
        for (int g = 0; g < 16; ++g) v += sh[g][threadIdx.x];
        if (c < split) out[c] = v;
        else out_hi[c - split] = v;
    }
}

__global__ void colsum_level_kernel(const float* __restrict__ X, long ldx, int M, int N, int chunk,
                                    float* __restrict__ out, long ldo, int split, float* __restrict__ out_hi) {
    __shared__ float sh[4][64];
    const int c = blockIdx.x * 64 + (threadIdx.x & 63);
    const int rg = threadIdx.x >> 6;
    const int r0 = blockIdx.y * chunk, r1 = min(M, r0 + chunk);
    float s = 0.f;
    if (c < N)
        for (int r = r0 + rg; r < r1; r += 4) s += X[(long)r * ldx + c];
    sh[rg][threadIdx.x & 63] = s;
    __syncthreads();
    if (rg == 0 && c < N) {
        const float v = ((sh[0][threadIdx.x] + sh[1][threadIdx.x]) + sh[2][threadIdx.x]) + sh[3][threadIdx.x];
        if (out_hi == nullptr) out[(long)blockIdx.y * ldo + c] = v;
        else if (c < split) out[c] = v;
        else out_hi[c - split] = v;
    }
}

// Optional launch timing (ptcg_profile_*): a HIP event pair around every
// timed launch (GEMMs, LayerNorm, Adam), recorded on the launch's own stream,
// with the launch's class and algorithmic amount (flops or bytes).
struct LaunchProf {
    bool on = false;
    int used = 0;
    std::vector<hipEvent_t> ev;
    std::vector<double> amount;
    std::vector<int> cls;
    double sum_ms[PROF_NCLASS] = {}, sum_amount[PROF_NCLASS] = {};
    int sum_n[PROF_NCLASS] = {};
};
LaunchProf g_prof;
int g_gemm_class = PROF_GEMM;

// products a launch executes: its share of the tiles, over the whole of K
// (split-K launches cover K across grid.z)
double launch_flops(const GemmArgs& g) {
    const double all = 2.0 * g.M * (double)g.N * g.K;
    if (!g.ntiles) return all;
    const double tiles = (double)pt_cdiv(g.M, BM) * pt_cdiv(g.N, BN);
    return all * g.ntiles / tiles;
}

template <bool AT, bool BT, int EPI, bool PARTIAL, bool DB, bool VEC>
void launch(const GemmArgs& g, dim3 grid, int k_chunk, long part_stride, hipStream_t s) {
    const int slot = pt_prof_open(s);
    if (VEC && g.dma)
        hipLaunchKernelGGL((gemm_f32_dma_kernel<AT, BT, EPI, PARTIAL, DB>), grid, dim3(NT), 0, s, g, k_chunk,
                           part_stride);
    else
        hipLaunchKernelGGL((gemm_f32_kernel<AT, BT, EPI, PARTIAL, DB, VEC>), grid, dim3(NT), 0, s, g, k_chunk,
                           part_stride);
    pt_prof_close(slot, g_gemm_class, launch_flops(g), s);
}

template <bool AT, bool BT, int EPI, bool PARTIAL, bool DB>
void launch_bf16(const GemmArgs& g, dim3 grid, int k_chunk, long part_stride, hipStream_t s) {
    const int slot = pt_prof_open(s);
    if (g.dma)
        hipLaunchKernelGGL((gemm_bf16_k16_kernel<AT, BT, EPI, PARTIAL, DB>), grid, dim3(NT), 0, s, g, k_chunk,
                           part_stride);
    else
        hipLaunchKernelGGL((gemm_bf16_kernel<AT, BT, EPI, PARTIAL>), grid, dim3(NT), 0, s, g, k_chunk, part_stride);
    pt_prof_close(slot, g_gemm_class, launch_flops(g), s);
}

// db: fused bias sums (A transposed, STORE epilogue, DMA kernel only)
template <bool AT, bool BT>
int launch_bf16_epi(const GemmArgs& g, dim3 grid, int k_chunk, long part_stride, bool partial, bool db,
                    hipStream_t s) {
    if (db) {
        PT_REQUIRE(AT && g.dma && g.epi == EPI_STORE, "gemm: bf16 bias sums need A transposed and the DMA kernel");
        if constexpr (AT) {
            if (partial) launch_bf16<AT, BT, EPI_STORE, true, true>(g, grid, k_chunk, part_stride, s);
            else launch_bf16<AT, BT, EPI_STORE, false, true>(g, grid, k_chunk, 0, s);
        }
        return PTCG_OK;
    }
    if (partial) {
        launch_bf16<AT, BT, EPI_STORE, true, false>(g, grid, k_chunk, part_stride, s);
        return PTCG_OK;
    }
    switch (g.epi) {
        case EPI_STORE: launch_bf16<AT, BT, EPI_STORE, false, false>(g, grid, k_chunk, 0, s); break;
        case EPI_BIAS: launch_bf16<AT, BT, EPI_BIAS, false, false>(g, grid, k_chunk, 0, s); break;
        case EPI_BIAS_GELU: launch_bf16<AT, BT, EPI_BIAS_GELU, false, false>(g, grid, k_chunk, 0, s); break;
        case EPI_BIAS_RESID: launch_bf16<AT, BT, EPI_BIAS_RESID, false, false>(g, grid, k_chunk, 0, s); break;
        case EPI_GELU_BWD: launch_bf16<AT, BT, EPI_GELU_BWD, false, false>(g, grid, k_chunk, 0, s); break;
        case EPI_BIAS_GELU_D: launch_bf16<AT, BT, EPI_BIAS_GELU_D, false, false>(g, grid, k_chunk, 0, s); break;
        case EPI_MUL: launch_bf16<AT, BT, EPI_MUL, false, false>(g, grid, k_chunk, 0, s); break;
        case EPI_AXPBY: launch_bf16<AT, BT, EPI_AXPBY, false, false>(g, grid, k_chunk, 0, s); break;
        case EPI_ACCUM: launch_bf16<AT, BT, EPI_ACCUM, false, false>(g, grid, k_chunk, 0, s); break;
        default: PT_REQUIRE(false, "gemm: bad epilogue %d", g.epi);
    }
    return PTCG_OK;
}

int launch_bf16_any(const GemmArgs& g, dim3 grid, int k_chunk, long part_stride, bool partial, bool db,
                    hipStream_t s) {
    const int code = (g.a_t ? 1 : 0) * 2 + (g.b_t ? 1 : 0);
    if (code == 0) return launch_bf16_epi<false, false>(g, grid, k_chunk, part_stride, partial, db, s);
    if (code == 1) return launch_bf16_epi<false, true>(g, grid, k_chunk, part_stride, partial, db, s);
    if (code == 3) return launch_bf16_epi<true, true>(g, grid, k_chunk, part_stride, partial, db, s);
    return launch_bf16_epi<true, false>(g, grid, k_chunk, part_stride, partial, db, s);
}

// split-K partial products (STORE into the workspace), optional bias sums
template <bool VEC>
void launch_partial(const GemmArgs& p, bool db, dim3 grid, int k_chunk, long part_stride, hipStream_t s) {
    const int code = (p.a_t ? 1 : 0) * 2 + (p.b_t ? 1 : 0);
    if (code == 3 && db) launch<true, true, EPI_STORE, true, true, VEC>(p, grid, k_chunk, part_stride, s);
    else if (code == 2 && db) launch<true, false, EPI_STORE, true, true, VEC>(p, grid, k_chunk, part_stride, s);
    else if (code == 3) launch<true, true, EPI_STORE, true, false, VEC>(p, grid, k_chunk, part_stride, s);
    else if (code == 1) launch<false, true, EPI_STORE, true, false, VEC>(p, grid, k_chunk, part_stride, s);
    else if (code == 0) launch<false, false, EPI_STORE, true, false, VEC>(p, grid, k_chunk, part_stride, s);
    else launch<true, false, EPI_STORE, true, false, VEC>(p, grid, k_chunk, part_stride, s);
}

template <bool AT, bool BT, bool VEC>
int launch_epi(const GemmArgs& g, dim3 grid, int k_chunk, hipStream_t s) {
    switch (g.epi) {
        case EPI_STORE: launch<AT, BT, EPI_STORE, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        case EPI_BIAS: launch<AT, BT, EPI_BIAS, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        case EPI_BIAS_GELU: launch<AT, BT, EPI_BIAS_GELU, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        case EPI_BIAS_RESID: launch<AT, BT, EPI_BIAS_RESID, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        case EPI_GELU_BWD: launch<AT, BT, EPI_GELU_BWD, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        case EPI_BIAS_GELU_D: launch<AT, BT, EPI_BIAS_GELU_D, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        case EPI_MUL: launch<AT, BT, EPI_MUL, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        case EPI_AXPBY: launch<AT, BT, EPI_AXPBY, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        case EPI_ACCUM: launch<AT, BT, EPI_ACCUM, false, false, VEC>(g, grid, k_chunk, 0, s); break;
        default: PT_REQUIRE(false, "gemm: bad epilogue %d", g.epi);
    }
    return PTCG_OK;
}

template <bool VEC>
int launch_full(const GemmArgs& g, bool db, dim3 grid, int k_chunk, hipStream_t s) {
    const int code = (g.a_t ? 1 : 0) * 2 + (g.b_t ? 1 : 0);
    if (db) {
        if (code == 3) launch<true, true, EPI_STORE, false, true, VEC>(g, grid, k_chunk, 0, s);
        else launch<true, false, EPI_STORE, false, true, VEC>(g, grid, k_chunk, 0, s);
        return PTCG_OK;
    }
    if (code == 0) return launch_epi<false, false, VEC>(g, grid, k_chunk, s);
    if (code == 1) return launch_epi<false, true, VEC>(g, grid, k_chunk, s);
    if (code == 3) return launch_epi<true, true, VEC>(g, grid, k_chunk, s);
    return launch_epi<true, false, VEC>(g, grid, k_chunk, s);
}

}  // namespace

bool pt_prof_active() { return g_prof.on; }

int pt_prof_gemm_class(int cls) {
    const int prev = g_gemm_class;
    g_gemm_class = cls;
    return prev;
}

// launches being captured into a graph are not timed (an event record would
// become a capture dependency, not a timestamp)
static bool prof_capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return s != nullptr && hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

int pt_prof_open(hipStream_t s) {
    if (!g_prof.on || g_prof.used * 2 + 1 >= (int)g_prof.ev.size() || prof_capturing(s)) return -1;
    (void)hipEventRecord(g_prof.ev[2 * g_prof.used], s);
    return g_prof.used++;
}

void pt_prof_close(int slot, int cls, double amount, hipStream_t s) {
    if (slot < 0) return;
    (void)hipEventRecord(g_prof.ev[2 * slot + 1], s);
    g_prof.cls[slot] = cls;
    g_prof.amount[slot] = amount;
}

extern "C" int ptcg_profile_begin(int max_launches) {
    PT_REQUIRE(max_launches > 0, "profile_begin: max_launches must be positive");
    for (auto e : g_prof.ev) (void)hipEventDestroy(e);
    g_prof.ev.assign(2 * (size_t)max_launches, nullptr);
    for (auto& e : g_prof.ev) PT_HIP(hipEventCreate(&e));
    g_prof.amount.assign(max_launches, 0.0);
    g_prof.cls.assign(max_launches, PROF_GEMM);
    g_prof.used = 0;
    g_prof.on = true;
    return PTCG_OK;
}

extern "C" int ptcg_profile_end(double* total_ms, int* launches, double* flops) {
    g_prof.on = false;
    for (int c = 0; c < PROF_NCLASS; ++c) {
        g_prof.sum_ms[c] = 0.0;
        g_prof.sum_amount[c] = 0.0;
        g_prof.sum_n[c] = 0;
    }
    for (int i = 0; i < g_prof.used; ++i) {
        PT_HIP(hipEventSynchronize(g_prof.ev[2 * i + 1]));
        float t = 0.f;
        PT_HIP(hipEventElapsedTime(&t, g_prof.ev[2 * i], g_prof.ev[2 * i + 1]));
        const int c = g_prof.cls[i];
        g_prof.sum_ms[c] += t;
        g_prof.sum_amount[c] += g_prof.amount[i];
        g_prof.sum_n[c]++;
    }
    if (total_ms) *total_ms = g_prof.sum_ms[PROF_GEMM];
    if (launches) *launches = g_prof.sum_n[PROF_GEMM];
    if (flops) *flops = g_prof.sum_amount[PROF_GEMM];
    for (auto e : g_prof.ev) (void)hipEventDestroy(e);
    g_prof.ev.clear();
    g_prof.used = 0;
    return PTCG_OK;
}

extern "C" int ptcg_profile_class(int cls, double* total_ms, int* launches, double* amount) {
    PT_REQUIRE(cls >= 0 && cls < PROF_NCLASS, "profile_class: class %d out of range", cls);
    if (total_ms) *total_ms = g_prof.sum_ms[cls];
    if (launches) *launches = g_prof.sum_n[cls];
    if (amount) *amount = g_prof.sum_amount[cls];
    return PTCG_OK;
}

// compute units of the current device (cached per device)
static int pt_cu_count() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cache[dev] = n;
    }
    return cache[dev];
}

// LDS-DMA kernels: every byte offset a tile can form (rows / columns up to
// one tile past the end) must fit the buffer instructions' 32-bit offsets
static bool dma_fits(int rows, int cols, long ld) {
    return ((long)rows + 2 * BM) * ld * 4 + ((long)cols + 2 * BM) * 4 < (1L << 31);
}
static bool dma_ok(const GemmArgs& g) {
    return dma_fits(g.a_t ? g.K : g.M, g.a_t ? g.M : g.K, g.lda) &&
           dma_fits(g.b_t ? g.K : g.N, g.b_t ? g.N : g.K, g.ldb);
}

// ---- bf16 storage (GemmArgs::bs)
// two DMA stages: measured faster than three or four at the trunk shapes
// (149 504 x {256, 768, 1024} x {256, 1024}): the smaller LDS footprint
// keeps more workgroups per CU, which hides the operand fetches better than
// a deeper pipeline per workgroup
constexpr int BS_NS = 2;
static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int EPI, bool OB>
static void launch_bs(const GemmArgs& f, dim3 grid, hipStream_t s) {
    hipLaunchKernelGGL((gemm_bs32_kernel<EPI, OB, BS_NS>), grid, dim3(NT), 0, s, f);
}

static int gemm_bs_nt(const GemmArgs& g, hipStream_t s) {
    PT_REQUIRE(g.K % 8 == 0 && g.lda % 8 == 0 && g.ldb % 8 == 0 && al16(g.A) && al16(g.B),
               "gemm (bf16 operands): K=%d, lda=%ld, ldb=%ld must be multiples of 8 and A, B 16 B aligned", g.K,
               g.lda, g.ldb);
    PT_REQUIRE(g.ldc % 4 == 0 && al16(g.C) && (!g.C2 || (g.ldc2 % 4 == 0 && al16(g.C2))),
               "gemm (bf16 operands): output leading dimensions must be multiples of 4, 16 B aligned");
    PT_REQUIRE(!g.Kdev && !g.dbias, "gemm (bf16 operands): no device K or bias sums in C = A B^T");
    GemmArgs f = g;   // float units for the DMA tile: 2 bf16 per float
    f.K = g.K / 2;
    f.lda = g.lda / 2;
    f.ldb = g.ldb / 2;
    f.dma = 1;
    f.tile0 = f.ntiles = f.tail_part = 0;
    PT_REQUIRE(dma_ok(f), "gemm (bf16 operands): operands exceed 2^31 bytes");
    const dim3 grid(pt_cdiv(g.M, BM) * pt_cdiv(g.N, BN));
    const int slot = pt_prof_open(s);
    const int code = g.epi * 2 + (g.obf ? 1 : 0);
    switch (code) {
        case EPI_STORE * 2: launch_bs<EPI_STORE, false>(f, grid, s); break;
        case EPI_STORE * 2 + 1: launch_bs<EPI_STORE, true>(f, grid, s); break;
        case EPI_BIAS * 2 + 1: launch_bs<EPI_BIAS, true>(f, grid, s); break;
        case EPI_BIAS_RESID * 2: launch_bs<EPI_BIAS_RESID, false>(f, grid, s); break;
        case EPI_BIAS_GELU_D * 2 + 1: launch_bs<EPI_BIAS_GELU_D, true>(f, grid, s); break;
        case EPI_MUL * 2 + 1: launch_bs<EPI_MUL, true>(f, grid, s); break;
        default:
            PT_REQUIRE(false, "gemm (bf16 operands): epilogue %d with %s output not built", g.epi,
                       g.obf ? "bf16" : "fp32");
    }
    pt_prof_close(slot, g_gemm_class, 2.0 * g.M * (double)g.N * g.K, s);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

static int gemm_bs_dw(const GemmArgs& g, float* ws, long ws_floats, hipStream_t s) {
    PT_REQUIRE(g.M % 8 == 0 && g.N % 8 == 0 && g.lda % 8 == 0 && g.ldb % 8 == 0 && al16(g.A) && al16(g.B),
               "gemm (bf16 weight gradient): M=%d, N=%d, lda=%ld, ldb=%ld must be multiples of 8, A and B 16 B "
               "aligned", g.M, g.N, g.lda, g.ldb);
    PT_REQUIRE(g.epi == EPI_STORE && !g.obf && !g.Mdev && g.ldc % 4 == 0 && al16(g.C),
               "gemm (bf16 weight gradient): fp32 STORE output with ldc a multiple of 4");
    const bool db = g.dbias != nullptr;
    if (g.M % 256 == 0 && g.N % 256 == 0) {
        // 256 x 256 tiles, one workgroup per CU: split the rows so the launch
        // has ~one block per CU, each >= 4 stages of 64 rows.  The bf16 step
        // at B = 2048: GEMM launches 9.66 -> 8.35 ms/step by events, the step
        // +4.6% against the 128 x 128 kernel (two A/B pairs on one box)
        const int tiles = (g.M / 256) * (g.N / 256);
        int splits = 1;
        const int cu = pt_cu_count() > 0 ? pt_cu_count() : 256;
        if (tiles < cu && g.K >= 8 * BKW) {
            splits = pt_cdiv(cu, tiles);
            const int max_splits = g.K / (4 * BKW);
            if (splits > max_splits) splits = max_splits;
            if (splits < 1) splits = 1;
        }
        const long part_stride = (long)g.M * g.ldc;
        const long per_split = part_stride + (db ? g.M : 0);
        if (splits > 1 && (ws == nullptr || (long)splits * per_split > ws_floats)) {
            const long fit = ws ? ws_floats / per_split : 0;
            splits = fit > 1 ? (int)fit : 1;
        }
        int k_chunk = g.K;
        if (splits > 1) {
            k_chunk = pt_cdiv(pt_cdiv(g.K, splits), BKW) * BKW;
            splits = pt_cdiv(g.K, k_chunk);
        }
        GemmArgs f = g;
        f.tile0 = f.ntiles = f.tail_part = 0;
        const dim3 grid(tiles, 1, splits);
        const size_t lds = 2 * 2 * 256 * BKW * sizeof(__bf16);
        static bool attr = false;
        if (!attr) {
            PT_HIP(hipFuncSetAttribute((const void*)gemm_bs_dw256_kernel<true, true>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            PT_HIP(hipFuncSetAttribute((const void*)gemm_bs_dw256_kernel<false, true>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            PT_HIP(hipFuncSetAttribute((const void*)gemm_bs_dw256_kernel<true, false>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            PT_HIP(hipFuncSetAttribute((const void*)gemm_bs_dw256_kernel<false, false>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            attr = true;
        }
        const int slot = pt_prof_open(s);
        if (splits > 1) {
            f.C = ws;
            if (db) hipLaunchKernelGGL((gemm_bs_dw256_kernel<true, true>), grid, dim3(512), lds, s, f, k_chunk, part_stride);
            else hipLaunchKernelGGL((gemm_bs_dw256_kernel<false, true>), grid, dim3(512), lds, s, f, k_chunk, part_stride);
        } else {
            if (db) hipLaunchKernelGGL((gemm_bs_dw256_kernel<true, false>), grid, dim3(512), lds, s, f, k_chunk, 0L);
            else hipLaunchKernelGGL((gemm_bs_dw256_kernel<false, false>), grid, dim3(512), lds, s, f, k_chunk, 0L);
        }
        pt_prof_close(slot, g_gemm_class, 2.0 * g.M * (double)g.N * g.K, s);
        PT_LAUNCH_CHECK();
        if (splits > 1) {
            launch_splitk_reduce<false>(g.C, g.ldc, ws, part_stride, splits, g.M, g.N, db ? g.dbias : nullptr, true, s);
            PT_LAUNCH_CHECK();
        }
        return PTCG_OK;
    }
    const int tiles = pt_cdiv(g.M, BM) * pt_cdiv(g.N, BN);
    // split the rows so the launch has ~256 blocks, each >= 4 stages of 64
    // rows: the blocks' weight gradients run on the step's side stream beside
    // the dX chain, and fewer, longer splits leave it more of the chip (the
    // bf16 step at B = 2048: 256 blocks +0.9%, 384 +0.7% against 512, two A/B
    // pairs on one box; 768 and 149.5k rows / 128 .. 256 no better)
    int splits = 1;
    if (tiles < 256 && g.K >= 8 * BKW) {
        splits = pt_cdiv(256, tiles);
        const int max_splits = g.K / (4 * BKW);
        if (splits > max_splits) splits = max_splits;
        if (splits < 1) splits = 1;
    }
    const long part_stride = (long)g.M * g.ldc;
    const long per_split = part_stride + (db ? g.M : 0);
    if (splits > 1 && (ws == nullptr || (long)splits * per_split > ws_floats)) {
        const long fit = ws ? ws_floats / per_split : 0;
        splits = fit > 1 ? (int)fit : 1;
    }
    int k_chunk = g.K;
    if (splits > 1) {
        k_chunk = pt_cdiv(pt_cdiv(g.K, splits), BKW) * BKW;
        splits = pt_cdiv(g.K, k_chunk);
    }
    GemmArgs f = g;
    f.tile0 = f.ntiles = f.tail_part = 0;
    const dim3 grid(tiles, 1, splits);
    const int slot = pt_prof_open(s);
    if (splits > 1) {
        f.C = ws;
        if (db) hipLaunchKernelGGL((gemm_bs_dw_kernel<true, true>), grid, dim3(NT), 0, s, f, k_chunk, part_stride);
        else hipLaunchKernelGGL((gemm_bs_dw_kernel<false, true>), grid, dim3(NT), 0, s, f, k_chunk, part_stride);
    } else {
        if (db) hipLaunchKernelGGL((gemm_bs_dw_kernel<true, false>), grid, dim3(NT), 0, s, f, k_chunk, 0L);
        else hipLaunchKernelGGL((gemm_bs_dw_kernel<false, false>), grid, dim3(NT), 0, s, f, k_chunk, 0L);
    }
    pt_prof_close(slot, g_gemm_class, 2.0 * g.M * (double)g.N * g.K, s);
    PT_LAUNCH_CHECK();
    if (splits > 1) {
        launch_splitk_reduce<false>(g.C, g.ldc, ws, part_stride, splits, g.M, g.N, db ? g.dbias : nullptr, true, s);
        PT_LAUNCH_CHECK();
    }
    return PTCG_OK;
}

// The residual product of a pre-LN block fused with the LayerNorm that reads
// its output (gemm_resid_ln_kernel).  g: EPI_BIAS_RESID with k-contiguous A
// (rows x K) and W (256 x K), fp32 output; fp32 operands, or bf16 ones (g.bs,
// K a multiple of 32).  pt_gemm_resid_ln_fits says whether g fits (the caller
// otherwise runs the product and the LayerNorm apart).  ybf: y in bf16.
static GemmArgs resid_ln_float_units(const GemmArgs& g) {
    GemmArgs f = g;
    if (g.bs) {   // 2 bf16 per float: the DMA tile's units
        f.K = g.K / 2;
        f.lda = g.lda / 2;
        f.ldb = g.ldb / 2;
    }
    return f;
}
bool pt_gemm_resid_ln_fits(const GemmArgs& g) {
    const uintptr_t al = (uintptr_t)g.A | (uintptr_t)g.B | (uintptr_t)g.C | (uintptr_t)g.R | (uintptr_t)g.bias |
                         (uintptr_t)(g.ldc * 4) | (uintptr_t)(g.ldr * 4) |
                         (uintptr_t)((g.lda | g.ldb) * (g.bs ? 2 : 4));
    const bool prec_ok = g.bs ? (g.K % 32 == 0 && g.lda % 8 == 0 && g.ldb % 8 == 0) : (g.prec == 0 && g.K % BK == 0);
    return g.N == RL_N && g.M > 0 && prec_ok && !g.a_t && !g.b_t && g.epi == EPI_BIAS_RESID && !g.obf && g.bias &&
           g.R && (al & 15) == 0 && !g.Kdev && dma_ok(resid_ln_float_units(g));
}
int pt_gemm_resid_ln(const GemmArgs& g, const float* lnw, const float* lnb, float* y, long ldy, float* mean,
                     float* rstd, hipStream_t s, int ybf) {
    PT_REQUIRE(g.A && g.B && g.C && lnw && lnb && y && mean && rstd, "gemm + layernorm: null operand");
    PT_REQUIRE(pt_gemm_resid_ln_fits(g),
               "gemm + layernorm: needs bias + residual with N = 256, K %% 16 == 0 (bf16 operands: %% 32), "
               "k-contiguous operands, 16 B aligned (M=%d, N=%d, K=%d)", g.M, g.N, g.K);
    PT_REQUIRE((((uintptr_t)lnw | (uintptr_t)lnb | (uintptr_t)y | (uintptr_t)(ldy * (ybf ? 2 : 4))) & 15) == 0,
               "gemm + layernorm: LayerNorm parameters and output need 16 B alignment");
    const GemmArgs f = resid_ln_float_units(g);
    // row tiles: 32 for fp32 operands (about 4.6 tiles per CU at 37.4k rows
    // instead of 2.3, so the last partial wave costs less: headline +0.4% on
    // one box), 128 for bf16 ones (every tile re-reads all of W from L2, so
    // larger row tiles halve that traffic: with the dX + LayerNorm backward
    // also on 128-row tiles the bf16 step at B = 2048 ran 1.2% faster than
    // on 64-row ones, two A/B pairs on one box; 32-row tiles were 2.8% slower
    // than 64-row ones)
    const dim3 blk(NT);
    const int slot = pt_prof_open(s);
    if (g.bs) {
        const dim3 grid(pt_cdiv(g.M, 128));
        if (ybf) hipLaunchKernelGGL((gemm_resid_ln_kernel<true, true, 128>), grid, blk, 0, s, f, lnw, lnb, y, ldy, mean, rstd);
        else hipLaunchKernelGGL((gemm_resid_ln_kernel<true, false, 128>), grid, blk, 0, s, f, lnw, lnb, y, ldy, mean, rstd);
    } else {
        const dim3 grid(pt_cdiv(g.M, 32));
        if (ybf) hipLaunchKernelGGL((gemm_resid_ln_kernel<false, true, 32>), grid, blk, 0, s, f, lnw, lnb, y, ldy, mean, rstd);
        else hipLaunchKernelGGL((gemm_resid_ln_kernel<false, false, 32>), grid, blk, 0, s, f, lnw, lnb, y, ldy, mean, rstd);
    }
    PT_LAUNCH_CHECK();
    pt_prof_close(slot, g_gemm_class, 2.0 * g.M * (double)g.N * g.K, s);
    return PTCG_OK;
}

// The bf16 dX product dy = dY W (dY rows x K, W^T copy 256 x K, both bf16)
// fused with the LayerNorm backward that reads dy (gemm_dx_lnbwd_kernel): dx
// (+ dres) fp32 and its bf16 copy dxh, dw / db from the per-workgroup partial
// rows by the fixed-order column sum.  x, dres, dx rows of 256 fp32.
bool pt_dx_lnbwd_fits(const GemmArgs& g) {
    return g.bs && g.N == RL_N && g.M > 0 && g.K % 32 == 0 && g.lda % 8 == 0 && g.ldb % 8 == 0 && !g.a_t &&
           !g.b_t && (((uintptr_t)g.A | (uintptr_t)g.B) & 15) == 0 && !g.Kdev && dma_ok(resid_ln_float_units(g));
}
int pt_dx_lnbwd(const GemmArgs& g, const float* x, const float* w, const float* mean, const float* rstd,
                const float* dres, float* dx, float* dxh, float* dw, float* db, float* ws, long ws_floats,
                hipStream_t s) {
    PT_REQUIRE(pt_dx_lnbwd_fits(g), "dX + layernorm bwd: needs bf16 operands, N = 256, K %% 32 == 0 (M=%d, K=%d)",
               g.M, g.K);
    PT_REQUIRE(g.A && g.B && x && w && mean && rstd && dx && dw && db && ws, "dX + layernorm bwd: null buffer");
    PT_REQUIRE((((uintptr_t)x | (uintptr_t)w | (uintptr_t)dx | (uintptr_t)dres | (uintptr_t)dxh) & 15) == 0,
               "dX + layernorm bwd: 16 B aligned rows needed");
    // 128-row tiles: W (256 x K bf16) is re-read from L2 once per tile
    const int blocks = pt_cdiv(g.M, 128);
    PT_REQUIRE((long)blocks * 2 * RL_N * 2 <= ws_floats, "dX + layernorm bwd: workspace too small");
    LnBwdArgs a{x, mean, rstd, w, dres, dx, reinterpret_cast<__bf16*>(dxh), ws};
    const GemmArgs f = resid_ln_float_units(g);
    const int slot = pt_prof_open(s);
    hipLaunchKernelGGL(gemm_dx_lnbwd_kernel<128>, dim3(blocks), dim3(NT), 0, s, f, a);
    PT_LAUNCH_CHECK();
    pt_prof_close(slot, g_gemm_class, 2.0 * g.M * (double)g.N * g.K, s);
    return pt_colsum2(ws, 2 * RL_N, blocks, 2 * RL_N, RL_N, dw, db, ws + (long)blocks * 2 * RL_N,
                      ws_floats - (long)blocks * 2 * RL_N, s);
}

// the device-decided balanced last wave: gemm_f32_dma_dtail_kernel, then
// dtail_reduce_kernel over its tail partials in ws
template <bool AT, bool BT, int EPI>
static void launch_dtail(const GemmArgs& g, int tiles, int S, float* ws, hipStream_t s) {
    const int slot = pt_prof_open(s);
    hipLaunchKernelGGL((gemm_f32_dma_dtail_kernel<AT, BT, EPI>), dim3(tiles + S), dim3(NT), 0, s, g, ws, S);
    pt_prof_close(slot, g_gemm_class, launch_flops(g), s);
    hipLaunchKernelGGL(dtail_reduce_kernel<EPI>, dim3(S * DTAIL_RED_WG), dim3(256), 0, s, g, (const float*)ws, S);
}
// the forward products (B not transposed) of the device-row-count layouts:
// in the backward the weight gradients on the side stream fill the CUs an
// unbalanced dX wave leaves idle (balancing them too measured no faster);
// false: not this product, nothing launched
static bool try_dtail(const GemmArgs& g, int tiles, int S, float* ws, hipStream_t s) {
    if (g.a_t || g.b_t) return false;
    switch (g.epi) {
        case EPI_BIAS: launch_dtail<false, false, EPI_BIAS>(g, tiles, S, ws, s); return true;
        case EPI_BIAS_RESID: launch_dtail<false, false, EPI_BIAS_RESID>(g, tiles, S, ws, s); return true;
        case EPI_BIAS_GELU_D: launch_dtail<false, false, EPI_BIAS_GELU_D>(g, tiles, S, ws, s); return true;
        default: return false;
    }
}

int pt_gemm(const GemmArgs& g0, float* ws, long ws_floats, hipStream_t s) {
    GemmArgs g = g0;
    PT_REQUIRE(g.M > 0 && g.N > 0 && g.K > 0, "gemm: empty shape %d x %d x %d", g.M, g.N, g.K);
    PT_REQUIRE(g.A && g.B && g.C, "gemm: null operand");
    if (g.bs) {
        PT_REQUIRE((!g.a_t && !g.b_t) || (g.a_t && g.b_t),
                   "gemm (bf16 operands): A and B both k-contiguous or both transposed");
        return g.a_t ? gemm_bs_dw(g, ws, ws_floats, s) : gemm_bs_nt(g, s);
    }
    PT_REQUIRE(!g.obf, "gemm: bf16 output needs bf16 operands");
    // 128-bit loads need the contiguous extent and the leading dimensions to be
    // multiples of 4 floats and 16 B aligned operands; otherwise scalar loads
    const bool vec = (g.a_t ? (g.M % 4 == 0) : (g.K % 4 == 0)) && (g.b_t ? (g.N % 4 == 0) : (g.K % 4 == 0)) &&
                     g.lda % 4 == 0 && g.ldb % 4 == 0 && ((uintptr_t)g.A & 15) == 0 &&
                     ((uintptr_t)g.B & 15) == 0;
    // bf16 products need the 128-bit operand path; other shapes stay fp32
    const bool bf = g.prec == 1 && vec;
    g.dma = vec && dma_ok(g);
    const int bk = bf && !g.dma ? BK2 : BK;
    const int tm = pt_cdiv(g.M, BM), tn = pt_cdiv(g.N, BN);
    const int tiles = tm * tn;
    // split K when the output is too small to fill the chip: long K in chunks
    // of >= 16 k-steps; short K (a few hundred rows, e.g. the weight gradients
    // of the per-sample MLPs at K = B) in chunks of >= 4 k-steps, so a handful
    // of tiles does not walk its whole K one stage at a time on a few CUs.
    // Products with a transposed A (the weight gradients, reduced over the
    // rows K) run on the step's side stream beside the dX chain: they aim at
    // a whole number of workgroups per CU, K / 128 rounded to the nearest
    // multiple of the CU count (1 .. 4 per CU), and take at most that many
    // (splits = target / tiles), so a launch alone has no partial last wave
    // and beside the dX chain leaves it the rest of the chip.  Measured
    // against 512 workgroups for every product (A/B pairs on one box each):
    // the CORE step at B = 512 (37.4k rows: 256 workgroups) +2.0% on one box
    // and even on another, the reference variant's step (82.4k rows: 768)
    // +0.6% and +0.5%; K / 128 unrounded (288 workgroups at 37.4k rows) was
    // as fast in the step but 60% slower alone, and 256 workgroups at 82.4k
    // rows 2.4% slower than 768.
    const int cu = pt_cu_count() > 0 ? pt_cu_count() : 256;
    // a weight gradient over a device row count (K here its host bound) on
    // the DMA kernel splits the device count as the rule gives for it (the
    // launch's splits cap it; later splits return): the launch takes the
    // rule's per-CU count rounded down on the bound, so that a device count
    // below the bound leaves few or no splits idle -- idle workgroups at the
    // end of a weight gradient running beside the dX chain delayed it (a
    // 256 x 256 weight gradient at 37.4k of 49.7k rows: 150 us with 500
    // workgroups of which 256 worked, 61 us with the 256 alone)
    const bool wsplit_ok = g.a_t && g.Kdev && !bf && vec && g.dma && (g.epi == EPI_STORE || g.epi == EPI_ACCUM);
    int splits = 1;
    if (g.a_t) {
        splits = pt_wgrad_splits(g.K, tiles, cu, bk, wsplit_ok);
    } else if (tiles < 512 && g.K >= 2 * bk * 4) {
        splits = pt_cdiv(512, tiles);
        const int min_steps = g.K >= 4 * bk * 16 ? 16 : 4;
        int max_splits = g.K / (bk * min_steps);
        if (splits > max_splits) splits = max_splits;
        if (splits < 1) splits = 1;
    }
    if (g.Mdev) splits = 1;   // device row counts: one pass (partials are sized by M)
    // bf16 output products (GemmArgs::obf) never reach this path; every fp32
    // epilogue is applied by the reduce when K is split
    PT_REQUIRE(!(g.dbias && !(g.a_t && g.epi == EPI_STORE)), "gemm: dbias needs a_t = 1 and the STORE epilogue");
    // the register-staged bf16 kernel leaves bias sums to the fp32 column sum
    // (from the unrounded dY); the DMA kernels sum the fp32 tiles in LDS
    const bool db = g.dbias != nullptr && (!bf || g.dma);
    long part_stride = (long)g.M * g.ldc;
    const long per_split = part_stride + (db ? g.M : 0);
    if (splits > 1 && (ws == nullptr || (long)splits * per_split > ws_floats)) {
        long fit = ws ? ws_floats / per_split : 0;
        splits = fit > 1 ? (int)fit : 1;
    }
    int k_chunk = g.K;
    if (splits > 1) splits = pt_split_chunks(g.K, splits, bk, &k_chunk);
    // the device-derived split count goes to the reduce as an int after the
    // partials (and bias partials)
    const int* sdev = nullptr;
    if (wsplit_ok && splits > 1 && (long)splits * per_split + 1 <= ws_floats) {
        g.wsplit = cu;
        sdev = reinterpret_cast<const int*>(ws + (long)splits * per_split);
    }
    dim3 grid(tn * tm, 1, splits);
    if (bf && g.dbias && !db) {
        // bias sums first: they read the fp32 dY, which the product does not modify
        PT_TRY(pt_colsum(g.A, g.lda, g.K, g.M, g.dbias, ws, ws_floats, s));
    }
    if (splits > 1) {
        GemmArgs p = g;
        p.C = ws;
        if (bf) PT_TRY(launch_bf16_any(p, grid, k_chunk, part_stride, true, db, s));
        else if (vec) launch_partial<true>(p, db, grid, k_chunk, part_stride, s);
        else launch_partial<false>(p, db, grid, k_chunk, part_stride, s);
        PT_LAUNCH_CHECK();
        const bool v4 = g.N % 4 == 0 && g.ldc % 4 == 0 && ((uintptr_t)g.C & 15) == 0;
        float* dbp = db ? g.dbias : nullptr;
        if (g.epi == EPI_ACCUM) {
            launch_splitk_reduce<true>(g.C, g.ldc, ws, part_stride, splits, g.M, g.N, dbp, v4, s, sdev);
        } else if (g.epi == EPI_STORE) {
            launch_splitk_reduce<false>(g.C, g.ldc, ws, part_stride, splits, g.M, g.N, dbp, v4, s, sdev);
        } else {
            const uintptr_t al = (uintptr_t)g.C | (uintptr_t)g.C2 | (uintptr_t)g.R | (uintptr_t)g.bias |
                                 (uintptr_t)((g.ldc | g.ldc2 | g.ldr) * 4);
            if (g.N % 4 == 0 && (al & 15) == 0) PT_TRY(launch_splitk_epi_reduce<true>(g, ws, part_stride, splits, s));
            else PT_TRY(launch_splitk_epi_reduce<false>(g, ws, part_stride, splits, s));
        }
        PT_LAUNCH_CHECK();
        return PTCG_OK;
    }
    // A device row count: the same balancing decided in the launches from the
    // count (whole tiles and tail partials, then the partials' fixed-order
    // sums through the epilogue), where the host's row bound allows a tail
    // (S < T) and leaves fewer than 8 tiles per CU
    if (g.Mdev && !g.Kdev && !db && !bf && g.dma && vec && ws != nullptr) {
        const int S = pt_cu_count();
        if (S > 0 && tiles > S && tiles < 8 * S && (long)S * BM * BN <= ws_floats && try_dtail(g, tiles, S, ws, s)) {
            PT_LAUNCH_CHECK();
            return PTCG_OK;
        }
    }
    // Balance the last wave: with T tiles on S CUs, T % S tail tiles would run
    // as a partial wave (e.g. 584 tiles = 2.28 per CU: the CUs holding 3 set
    // the time).  Run the first T - T % S tiles whole and split the tail's K
    // across the idle CUs, then reduce the tail partials in a fixed order.
    // Worth its two extra launches only while a CU holds few tiles (T < 4 S).
    if (!db && !g.Mdev && ws != nullptr) {
        const int S = pt_cu_count();
        const int R = S > 0 ? tiles % S : 0;
        const int ksteps = pt_cdiv(g.K, bk);
        int s2 = R ? S / R : 0;
        if (s2 > ksteps / 2) s2 = ksteps / 2;
        if (tiles > S && tiles < 4 * S && R != 0 && s2 >= 2 && (long)s2 * R * BM * BN <= ws_floats) {
            const int kc = pt_cdiv(pt_cdiv(g.K, s2), bk) * bk;
            s2 = pt_cdiv(g.K, kc);
            GemmArgs a = g;
            a.tile0 = 0;
            a.ntiles = tiles - R;
            const dim3 ga(tiles - R, 1, 1);
            if (bf) PT_TRY(launch_bf16_any(a, ga, g.K, 0, false, false, s));
            else PT_TRY(vec ? launch_full<true>(a, false, ga, g.K, s) : launch_full<false>(a, false, ga, g.K, s));
            PT_LAUNCH_CHECK();
            GemmArgs p = g;
            p.C = ws;
            p.tile0 = tiles - R;
            p.ntiles = R;
            p.tail_part = 1;
            const dim3 gp(R, 1, s2);
            if (bf) PT_TRY(launch_bf16_any(p, gp, kc, 0, true, false, s));
            else if (vec) launch_partial<true>(p, false, gp, kc, 0, s);
            else launch_partial<false>(p, false, gp, kc, 0, s);
            PT_LAUNCH_CHECK();
            GemmArgs t = g;
            t.tile0 = tiles - R;
            t.ntiles = R;
            const dim3 gr(pt_cdiv((long)R * BM * BN, 256));
            switch (g.epi) {
                case EPI_STORE: hipLaunchKernelGGL(tail_reduce_kernel<EPI_STORE>, gr, dim3(256), 0, s, t, ws, s2); break;
                case EPI_BIAS: hipLaunchKernelGGL(tail_reduce_kernel<EPI_BIAS>, gr, dim3(256), 0, s, t, ws, s2); break;
                case EPI_BIAS_GELU: hipLaunchKernelGGL(tail_reduce_kernel<EPI_BIAS_GELU>, gr, dim3(256), 0, s, t, ws, s2); break;
                case EPI_BIAS_RESID: hipLaunchKernelGGL(tail_reduce_kernel<EPI_BIAS_RESID>, gr, dim3(256), 0, s, t, ws, s2); break;
                case EPI_GELU_BWD: hipLaunchKernelGGL(tail_reduce_kernel<EPI_GELU_BWD>, gr, dim3(256), 0, s, t, ws, s2); break;
                case EPI_BIAS_GELU_D: hipLaunchKernelGGL(tail_reduce_kernel<EPI_BIAS_GELU_D>, gr, dim3(256), 0, s, t, ws, s2); break;
                case EPI_MUL: hipLaunchKernelGGL(tail_reduce_kernel<EPI_MUL>, gr, dim3(256), 0, s, t, ws, s2); break;
                case EPI_AXPBY: hipLaunchKernelGGL(tail_reduce_kernel<EPI_AXPBY>, gr, dim3(256), 0, s, t, ws, s2); break;
                case EPI_ACCUM: hipLaunchKernelGGL(tail_reduce_kernel<EPI_ACCUM>, gr, dim3(256), 0, s, t, ws, s2); break;
                default: PT_REQUIRE(false, "gemm: bad epilogue %d", g.epi);
            }
            PT_LAUNCH_CHECK();
            return PTCG_OK;
        }
    }
    if (bf) PT_TRY(launch_bf16_any(g, grid, k_chunk, 0, false, db, s));
    else PT_TRY(vec ? launch_full<true>(g, db, grid, k_chunk, s) : launch_full<false>(g, db, grid, k_chunk, s));
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

namespace {
template <bool AT, bool BT>
int launch_grouped(const GroupedGemm* d, const int* ig, int items, int epi, int partial, hipStream_t s) {
    const dim3 grid(items), blk(NT);
    if (partial && epi == EPI_STORE)
        hipLaunchKernelGGL((gemm_f32_dma_grouped_kernel<AT, BT, EPI_STORE, true>), grid, blk, 0, s, d, ig);
    else if (!partial && epi == EPI_STORE)
        hipLaunchKernelGGL((gemm_f32_dma_grouped_kernel<AT, BT, EPI_STORE, false>), grid, blk, 0, s, d, ig);
    else if (!partial && epi == EPI_AXPBY)
        hipLaunchKernelGGL((gemm_f32_dma_grouped_kernel<AT, BT, EPI_AXPBY, false>), grid, blk, 0, s, d, ig);
    else
        PT_REQUIRE(false, "gemm_grouped: epilogue %d (partial %d) not supported", epi, partial);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
}  // namespace

int pt_gemm_grouped(const GroupedGemm* d_groups, const int* d_item_group, int items, int a_t, int b_t, int epi,
                    int partial, double flops, hipStream_t s) {
    PT_REQUIRE(d_groups && d_item_group && items > 0, "gemm_grouped: empty launch");
    const int code = (a_t ? 2 : 0) + (b_t ? 1 : 0);
    const int slot = pt_prof_open(s);
    int r;
    if (code == 0) r = launch_grouped<false, false>(d_groups, d_item_group, items, epi, partial, s);
    else if (code == 1) r = launch_grouped<false, true>(d_groups, d_item_group, items, epi, partial, s);
    else if (code == 2) r = launch_grouped<true, false>(d_groups, d_item_group, items, epi, partial, s);
    else r = launch_grouped<true, true>(d_groups, d_item_group, items, epi, partial, s);
    pt_prof_close(slot, g_gemm_class, flops, s);
    return r;
}

int pt_grouped_reduce(const GroupedGemm* d_groups, const int* d_chunk_group, const int* d_chunk_first, int chunks,
                      hipStream_t s) {
    PT_REQUIRE(d_groups && d_chunk_group && d_chunk_first && chunks > 0, "grouped_reduce: empty launch");
    hipLaunchKernelGGL(grouped_reduce_kernel, dim3(chunks), dim3(256), 0, s, d_groups, d_chunk_group, d_chunk_first);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

int pt_linear_fwd(const float* X, const float* W, const float* b, float* Y, int rows, int in,
                  int out, int epi, const float* R, float* Y2, hipStream_t s) {
    GemmArgs g{};
    g.M = rows; g.N = out; g.K = in;
    g.A = X; g.lda = in; g.a_t = 0;
    g.B = W; g.ldb = in; g.b_t = 0;
    g.C = Y; g.ldc = out;
    g.bias = b; g.R = R; g.ldr = out; g.C2 = Y2; g.ldc2 = out;
    g.epi = epi;
    if ((epi == EPI_BIAS || epi == EPI_BIAS_GELU || epi == EPI_BIAS_RESID || epi == EPI_BIAS_GELU_D) && b == nullptr)
        g.epi = (epi == EPI_BIAS) ? EPI_STORE : epi;
    PT_REQUIRE(!(g.epi == EPI_BIAS_GELU || g.epi == EPI_BIAS_RESID || g.epi == EPI_BIAS_GELU_D) || b != nullptr,
               "linear_fwd: epilogue %d needs a bias", epi);
    return pt_gemm(g, nullptr, 0, s);
}

int pt_linear_dx(const float* dY, const float* W, float* dX, int rows, int in, int out, int epi,
                 const float* R, hipStream_t s) {
    GemmArgs g{};
    g.M = rows; g.N = in; g.K = out;
    g.A = dY; g.lda = out; g.a_t = 0;
    g.B = W; g.ldb = in; g.b_t = 1;
    g.C = dX; g.ldc = in;
    g.R = R; g.ldr = in;
    g.epi = epi;
    return pt_gemm(g, nullptr, 0, s);
}

int pt_linear_dw(const float* dY, const float* X, float* dW, float* db, int rows, int in, int out,
                 float* ws, long ws_floats, hipStream_t s) {
    GemmArgs g{};
    g.M = out; g.N = in; g.K = rows;
    g.A = dY; g.lda = out; g.a_t = 1;
    g.B = X; g.ldb = in; g.b_t = 1;
    g.C = dW; g.ldc = in;
    g.epi = EPI_STORE;
    g.dbias = db;
    return pt_gemm(g, ws, ws_floats, s);
}

int pt_colsum2(const float* X, long ldx, int M, int N, int split, float* out_lo, float* out_hi,
               float* ws, long ws_floats, hipStream_t s) {
    PT_REQUIRE(M > 0 && N > 0, "colsum: empty shape %d x %d", M, N);
    if (M <= 4096) {
        // one launch: a workgroup per 64 columns, sixteen row groups of a
        // column summed in a fixed order (the per-block partial rows of the
        // LayerNorm backward and the small bias sums: two launches of a few
        // rows each were bound by their launch latency)
        hipLaunchKernelGGL(colsum_one_kernel, dim3(pt_cdiv(N, 64)), dim3(1024), 0, s, X, ldx, M, N, out_lo,
                           out_hi ? split : N, out_hi ? out_hi : out_lo + N);
        PT_LAUNCH_CHECK();
        return PTCG_OK;
    }
    int slices = pt_cdiv(M, 64);
    if (slices > 256) slices = 256;
    const int chunk = pt_cdiv(M, slices);
    slices = pt_cdiv(M, chunk);
    PT_REQUIRE(ws != nullptr && (long)slices * N <= ws_floats, "colsum: workspace too small (%d x %d)", slices, N);
    hipLaunchKernelGGL(colsum_level_kernel, dim3(pt_cdiv(N, 64), slices), dim3(256), 0, s, X, ldx, M, N, chunk,
                       ws, (long)N, 0, nullptr);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(colsum_level_kernel, dim3(pt_cdiv(N, 64), 1), dim3(256), 0, s, ws, (long)N, slices, N,
                       slices, out_lo, 0L, out_hi ? split : N, out_hi ? out_hi : out_lo + N);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

int pt_colsum(const float* X, long ldx, int M, int N, float* out, float* ws, long ws_floats,
              hipStream_t s) {
    return pt_colsum2(X, ldx, M, N, N, out, nullptr, ws, ws_floats, s);
}
