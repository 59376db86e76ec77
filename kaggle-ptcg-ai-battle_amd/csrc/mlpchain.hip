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
