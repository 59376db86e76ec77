// The per-sample MLPs ahead of the trunk in one launch: the global MLP
// g = W2 gelu(W1 global_f + b1) + b2, the decision MLP d = W4 gelu(W3 dec_in
// + b3) + b4 and the broadcast product bc = Wb [g | d] + bb (reference:
// ptcg/rl/model.py:134-142 global_mlp / dec_mlp / bcast, used at :223-235).
//
// At B samples these are five products of B rows (about 0.12 GFLOP at B =
// 512): as separate GEMM launches they form a chain of ten or more dependent
// launches whose latency, not their arithmetic, sets when the trunk can start.
// Here a workgroup takes MC_R samples through all five layers with the
// activations in LDS; each output element is a 16-lane group's fp32 dot
// product (fused multiply-adds over each lane's k in order, then a fixed
// butterfly over the group: deterministic), the weights read as contiguous
// 256-byte runs of a row, a pass's loads all in flight together.  It writes what the GEMM launches wrote
// for the backward: gelu'(z) and gelu(z) of both hidden layers, gd = [g | d]
// and bc.
#include "model.h"

namespace {

constexpr int MC_R = 4;      // samples per workgroup
constexpr int MC_T = 512;    // threads per workgroup
constexpr int MC_LG = 16;    // lanes that split one column's k
constexpr int MC_J = 4;      // columns per lane group and pass
constexpr int MC_KB = 8;     // weight float4s per lane and column loaded together (k chunks of 512)
constexpr int MC_COLS = MC_T / MC_LG * MC_J;   // columns per pass of the workgroup
static_assert(MC_R <= MC_LG, "lane r of a group finishes row r");

// Z = X W^T + b for the workgroup's MC_R rows: X in LDS (MC_R x in, row
// stride ldx), W (out, in) row-major.  Columns go MC_COLS at a time, MC_J to
// each 16-lane group of the eight waves; the group's lanes split k (lane l of
// the group takes float4s l, l + 16, ...: a group reads 256 contiguous bytes
// of a weight row per load, and every load of the pass is issued before the
// first product), then sum their partial dot products over the group in a
// fixed butterfly order, and lane r of the group finishes row r.  (One
// workgroup per CU, two waves per SIMD: the weights of a pass, 128 registers
// a lane, are all in flight at once.)  gelu: Y = gelu'(z), Y2 =
// gelu(z), L = gelu(z); else Y = z, L = z.  Global rows past nrows are not
// stored (their LDS rows are zeros in, finite values out).
__device__ __forceinline__ void mc_dense(const float* X, int ldx, int in, const float* __restrict__ W, const float* __restrict__ b,
                         int out, bool gelu, float* __restrict__ Y, long ldy, float* __restrict__ Y2, long ldy2,
                         float* L, int ldl, int row0, int nrows) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gl = lane % MC_LG, grp = lane / MC_LG;
    const int n4 = in / 4, ldx4 = ldx / 4;
    const float4* X4 = reinterpret_cast<const float4*>(X);
    for (int jb = 0; jb < out; jb += MC_COLS) {
        int j[MC_J];
        const float4* w[MC_J];
        float acc[MC_J][MC_R];
#pragma unroll
        for (int c = 0; c < MC_J; ++c) {
            j[c] = jb + c * (MC_T / MC_LG) + (64 / MC_LG) * wave + grp;
            w[c] = reinterpret_cast<const float4*>(W + (long)(j[c] < out ? j[c] : 0) * in);
#pragma unroll
            for (int r = 0; r < MC_R; ++r) acc[c][r] = 0.f;
        }
        for (int kc = 0; kc < n4; kc += MC_LG * MC_KB) {
            float4 wv[MC_J][MC_KB];
#pragma unroll
            for (int c = 0; c < MC_J; ++c)
#pragma unroll
                for (int u = 0; u < MC_KB; ++u) {
                    const int k4 = kc + u * MC_LG + gl;
                    wv[c][u] = j[c] < out && k4 < n4 ? w[c][k4] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
            for (int u = 0; u < MC_KB; ++u) {
                const int k4 = kc + u * MC_LG + gl;
                if (k4 < n4) {
#pragma unroll
                    for (int r = 0; r < MC_R; ++r) {
                        const float4 xv = X4[r * ldx4 + k4];
#pragma unroll
                        for (int c = 0; c < MC_J; ++c) {
                            acc[c][r] = fmaf(xv.x, wv[c][u].x, acc[c][r]);
                            acc[c][r] = fmaf(xv.y, wv[c][u].y, acc[c][r]);
                            acc[c][r] = fmaf(xv.z, wv[c][u].z, acc[c][r]);
                            acc[c][r] = fmaf(xv.w, wv[c][u].w, acc[c][r]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int o = MC_LG / 2; o > 0; o >>= 1)
#pragma unroll
            for (int c = 0; c < MC_J; ++c)
#pragma unroll
                for (int r = 0; r < MC_R; ++r) acc[c][r] += __shfl_xor(acc[c][r], o, 64);
#pragma unroll
        for (int c = 0; c < MC_J; ++c) {
            if (j[c] >= out) continue;
            const float bj = b[j[c]];
#pragma unroll
            for (int r = 0; r < MC_R; ++r) {
                if (gl != r) continue;
                const float z = acc[c][r] + bj;
                float v = z;
                if (gelu) {
                    float g, gd;
                    pt_gelu_both(z, g, gd);
                    v = g;
                    if (r < nrows) {
                        Y[(long)(row0 + r) * ldy + j[c]] = gd;
                        Y2[(long)(row0 + r) * ldy2 + j[c]] = g;
                    }
                } else if (r < nrows) {
                    Y[(long)(row0 + r) * ldy + j[c]] = z;
                }
                if (L) L[r * ldl + j[c]] = v;
            }
        }
    }
}

// rows [row0, row0 + MC_R) of src (ld w) into LDS (MC_R x w), zeros past nrows
__device__ void mc_load(float* dst, const float* __restrict__ src, int w, int row0, int nrows) {
    for (int i = threadIdx.x; i < MC_R * w; i += MC_T) {
        const int r = i / w, k = i - r * w;
        dst[i] = r < nrows ? src[(long)(row0 + r) * w + k] : 0.f;
    }
}

__global__ __launch_bounds__(MC_T) void mlp_chain_fwd_kernel(const MlpChain a) {
    extern __shared__ __align__(16) float mc_smem[];
    const int lx = a.gf > a.din ? a.gf : a.din, lh = a.G > a.H ? a.G : a.H, bin = a.G + a.H;
    float* xin = mc_smem;               // MC_R x lx
    float* hid = xin + MC_R * lx;       // MC_R x lh
    float* gdl = hid + MC_R * lh;       // MC_R x bin: [g | d]
    const int row0 = blockIdx.x * MC_R;
    const int nrows = a.N - row0 < MC_R ? a.N - row0 : MC_R;
    // global MLP
    mc_load(xin, a.glob_in, a.gf, row0, nrows);
    __syncthreads();
    mc_dense(xin, a.gf, a.gf, a.g1w, a.g1b, a.G, true, a.g1, a.G, a.g1a, a.G, hid, a.G, row0, nrows);
    __syncthreads();
    mc_dense(hid, a.G, a.G, a.g2w, a.g2b, a.G, false, a.gd, bin, nullptr, 0, gdl, bin, row0, nrows);
    __syncthreads();
    // decision MLP
    mc_load(xin, a.dec_in, a.din, row0, nrows);
    __syncthreads();
    mc_dense(xin, a.din, a.din, a.d1w, a.d1b, a.H, true, a.d1, a.H, a.d1a, a.H, hid, a.H, row0, nrows);
    __syncthreads();
    mc_dense(hid, a.H, a.H, a.d2w, a.d2b, a.H, false, a.gd + a.G, bin, nullptr, 0, gdl + a.G, bin, row0, nrows);
    __syncthreads();
    // broadcast product over [g | d]
    mc_dense(gdl, bin, bin, a.bcw, a.bcb, a.D, false, a.bc, a.D, nullptr, 0, nullptr, 0, row0, nrows);
}

long mc_smem_bytes(const MlpChain& a) {
    const int lx = a.gf > a.din ? a.gf : a.din, lh = a.G > a.H ? a.G : a.H;
    return 4L * MC_R * (lx + lh + a.G + a.H);
}

}  // namespace

bool pt_mlp_chain_fits(const MlpChain& a) {
    const float* w[] = {a.g1w, a.g2w, a.d1w, a.d2w, a.bcw};
    for (const float* p : w)
        if (p == nullptr || ((uintptr_t)p & 15) != 0) return false;
    return a.N >= 1 && a.gf % 4 == 0 && a.G % 4 == 0 && a.din % 4 == 0 && a.H % 4 == 0 && a.D >= 1 &&
           mc_smem_bytes(a) <= 64 * 1024;
}

int pt_mlp_chain_fwd(const MlpChain& a, hipStream_t s) {
    PT_REQUIRE(pt_mlp_chain_fits(a), "mlp_chain: widths %d / %d / %d / %d / %d or weight alignment not supported",
               a.gf, a.G, a.din, a.H, a.D);
    PT_REQUIRE(a.glob_in && a.dec_in && a.g1b && a.g2b && a.d1b && a.d2b && a.bcb && a.g1 && a.g1a && a.gd && a.d1 &&
                   a.d1a && a.bc,
               "mlp_chain: null pointer");
    hipLaunchKernelGGL(mlp_chain_fwd_kernel, dim3(pt_cdiv(a.N, MC_R)), dim3(MC_T), (size_t)mc_smem_bytes(a), s, a);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

// The backward's dX products of the same chain in one launch (reference:
// the autograd of ptcg/rl/model.py:223-235): dgd += dbc Wb, dd1 = (dgd[:, G:]
// W4) * gelu'(z3), ddec = dd1 W3, dg1 = (dgd[:, :G] W2) * gelu'(z1).  A
// workgroup takes MB_R samples; per product a thread owns an output column j
// for all MB_R rows and runs over the reduction index in order (the weight
// row segments W[o][j..] of consecutive threads are contiguous), MB_B weights
// in flight at once.  Deterministic; writes dgd, dd1, ddec and dg1 as the
// separate products did.
namespace {

constexpr int MB_R = 4;      // samples per workgroup
constexpr int MB_T = 512;    // threads per workgroup
constexpr int MB_B = 32;     // weights per thread loaded together

// Y[r][j] (+)= sum_o X[r][o] W[o][j] for the workgroup's MB_R rows: X in LDS
// (MB_R x nin at row stride ldx), W (nin, nout) row-major; mul: Y = sum *
// M[row][j] (M at row stride ldm); acc: Y = Yold + sum; L: the result for the
// next product (LDS, row stride ldl)
__device__ __forceinline__ void mb_dense(const float* X, int ldx, int nin, const float* __restrict__ W, int nout,
                                         float* __restrict__ Y, long ldy, bool acc, const float* __restrict__ M,
                                         long ldm, float* L, int ldl, int row0, int nrows) {
    for (int j = threadIdx.x; j < nout; j += MB_T) {
        float s[MB_R];
#pragma unroll
        for (int r = 0; r < MB_R; ++r) s[r] = 0.f;
        for (int ob = 0; ob < nin; ob += MB_B) {
            float wv[MB_B];
#pragma unroll
            for (int u = 0; u < MB_B; ++u) wv[u] = ob + u < nin ? W[(long)(ob + u) * nout + j] : 0.f;
#pragma unroll
            for (int u = 0; u < MB_B; ++u) {
                if (ob + u >= nin) break;
#pragma unroll
                for (int r = 0; r < MB_R; ++r) s[r] = fmaf(X[r * ldx + ob + u], wv[u], s[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < MB_R; ++r) {
            float v = s[r];
            if (r < nrows) {
                float* y = Y + (long)(row0 + r) * ldy + j;
                if (acc) v = *y + v;
                if (M) v *= M[(long)(row0 + r) * ldm + j];
                *y = v;
            }
            if (L) L[r * ldl + j] = v;
        }
    }
}

__device__ __forceinline__ void mb_load(float* dst, int ldd, const float* __restrict__ src, long lds, int w, int row0,
                                        int nrows) {
    for (int i = threadIdx.x; i < MB_R * w; i += MB_T) {
        const int r = i / w, k = i - r * w;
        dst[r * ldd + k] = r < nrows ? src[(long)(row0 + r) * lds + k] : 0.f;
    }
}

__global__ __launch_bounds__(MB_T) void mlp_chain_bwd_kernel(const MlpChainBwd a) {
    extern __shared__ __align__(16) float mb_smem[];
    const int bin = a.G + a.H;
    float* dbc = mb_smem;                 // MB_R x D
    float* dgd = dbc + MB_R * a.D;        // MB_R x bin (after the broadcast product)
    float* dd1 = dgd + MB_R * bin;        // MB_R x H
    const int row0 = blockIdx.x * MB_R;
    const int nrows = a.N - row0 < MB_R ? a.N - row0 : MB_R;
    mb_load(dbc, a.D, a.dbc, a.D, a.D, row0, nrows);
    __syncthreads();
    // dgd += dbc Wb  (Wb: D x bin)
    mb_dense(dbc, a.D, a.D, a.bcw, bin, a.dgd, bin, true, nullptr, 0, dgd, bin, row0, nrows);
    __syncthreads();
    // dd1 = (dgd[:, G:] W4) * d1, W4: H x H;  dg1 = (dgd[:, :G] W2) * g1, W2: G x G
    mb_dense(dgd + a.G, bin, a.H, a.d2w, a.H, a.dd1, a.H, false, a.d1, a.H, dd1, a.H, row0, nrows);
    mb_dense(dgd, bin, a.G, a.g2w, a.G, a.dg1, a.G, false, a.g1, a.G, nullptr, 0, row0, nrows);
    __syncthreads();
    // ddec = dd1 W3, W3: H x din
    mb_dense(dd1, a.H, a.H, a.d1w, a.din, a.ddec, a.din, false, nullptr, 0, nullptr, 0, row0, nrows);
}

}  // namespace

int pt_mlp_chain_bwd(const MlpChainBwd& a, hipStream_t s) {
    PT_REQUIRE(a.N >= 1 && a.G >= 1 && a.H >= 1 && a.din >= 1 && a.D >= 1, "mlp_chain_bwd: empty widths");
    PT_REQUIRE(a.dbc && a.bcw && a.g2w && a.d2w && a.d1w && a.g1 && a.d1 && a.dgd && a.dg1 && a.dd1 && a.ddec,
               "mlp_chain_bwd: null pointer");
    const long smem = 4L * MB_R * (a.D + a.G + a.H + a.H);
    PT_REQUIRE(smem <= 64 * 1024, "mlp_chain_bwd: widths %d / %d / %d exceed LDS", a.D, a.G, a.H);
    hipLaunchKernelGGL(mlp_chain_bwd_kernel, dim3(pt_cdiv(a.N, MB_R)), dim3(MB_T), (size_t)smem, s, a);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
