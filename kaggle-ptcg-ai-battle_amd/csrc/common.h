// Shared helpers for the PTCG HIP kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "../../include/ptcg_amd.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));
// global-address-space views (lets the compiler emit global_load, not flat_load)
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) floatx4 gfloatx4;
__device__ __forceinline__ float4 ld_g4(const gfloat* p) {
    const floatx4 v = *(const gfloatx4*)p;
    return make_float4(v[0], v[1], v[2], v[3]);
}

// ---------------------------------------------------------------- errors
void ptcg_set_error(const char* fmt, ...);

#define PT_HIP(call)                                                        \
    do {                                                                    \
        hipError_t _e = (call);                                             \
        if (_e != hipSuccess) {                                             \
            ptcg_set_error("%s:%d %s: %s", __FILE__, __LINE__, #call,       \
                           hipGetErrorString(_e));                          \
            return PTCG_ERR_HIP;                                            \
        }                                                                   \
    } while (0)

#define PT_REQUIRE(cond, ...)                                               \
    do {                                                                    \
        if (!(cond)) {                                                      \
            ptcg_set_error(__VA_ARGS__);                                    \
            return PTCG_ERR_ARG;                                            \
        }                                                                   \
    } while (0)

#define PT_TRY(expr)                                                        \
    do {                                                                    \
        int _r = (expr);                                                    \
        if (_r != PTCG_OK) return _r;                                       \
    } while (0)

// launch then check the launch status
#define PT_LAUNCH_CHECK()  PT_HIP(hipGetLastError())

static inline int pt_cdiv(long a, long b) { return (int)((a + b - 1) / b); }

// Launch timing for ptcg_profile_*: pt_prof_open records a start event on the
// stream and returns a slot (-1 when no profile is open); pt_prof_close
// records the end event with the launch's class and algorithmic amount
// (flops for GEMMs, HBM bytes for the others).
enum PtProfClass { PROF_GEMM = 0, PROF_LN_FWD = 1, PROF_LN_BWD = 2, PROF_ADAM_NORM = 3, PROF_ADAM_UPDATE = 4,
                   PROF_MUON = 5, PROF_MUON_GEMM = 6, PROF_GATHER = 7, PROF_PPO = 8, PROF_NCLASS = 9 };
int pt_prof_open(hipStream_t s);
void pt_prof_close(int slot, int cls, double amount, hipStream_t s);
// class recorded for GEMM launches (PROF_GEMM unless a caller such as the
// Muon step files its products separately); returns the previous class
int pt_prof_gemm_class(int cls);
// true while a launch profile is open: concurrent streams would overlap the
// timed launches, so callers that fork work onto a second stream keep it on
// the launch stream instead
bool pt_prof_active();

// ---------------------------------------------------------------- device math
// Exact (erf) GELU, torch nn.GELU() default; the reference's pt_gelu_fwd/bwd
// (ptcg_kernels.cuh:111-128) computes the same function and derivative.
// GELU and its derivative from one branch-free erf: Abramowitz & Stegun,
// Handbook of Mathematical Functions, formula 7.1.26 (|error| <= 1.5e-7 on
// [0, inf)), 1 - erf(x) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) e^(-x^2),
// t = 1 / (1 + p x), x = |z| / sqrt 2, whose e^(-x^2) = e^(-z^2/2) is also
// the normal density's exponential in gelu'(z) = Phi(z) + z phi(z).  t comes
// from v_rcp_f32 (1 ulp) in place of an IEEE division.  The GEMM epilogues
// that apply it run after the products and are bound by their VALU work:
// libm's erf (branches over |x| ranges) and a separate expf for the density
// cost the fp32 FFN1 product with this epilogue 30 us per launch more than
// the same-shape FFN2 dX product with a multiply epilogue.
__device__ __forceinline__ void pt_gelu_both(float z, float& g, float& gd) {
    const float x = fabsf(z) * 0.70710678118654752f;
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * x);
    const float poly =
        t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
    const float e = __expf(-x * x);
    const float q = poly * e;   // 1 - erf(|z| / sqrt 2)
    const float cdf = z >= 0.f ? 1.0f - 0.5f * q : 0.5f * q;
    g = z * cdf;
    gd = cdf + z * (0.3989422804014327f * e);
}
__device__ __forceinline__ float pt_gelu(float x) {
    float g, gd;
    pt_gelu_both(x, g, gd);
    return g;
}
__device__ __forceinline__ float pt_gelu_grad(float x) {
    float g, gd;
    pt_gelu_both(x, g, gd);
    return gd;
}
// the mixed-precision variant's stored activations (bf16 outputs): the same
// function (its error is far below the 2^-9 rounding of the stored value)
__device__ __forceinline__ void pt_gelu_both_bf(float z, float& g, float& gd) { pt_gelu_both(z, g, gd); }

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC'11), restated from the paper: 10 rounds of
// (hi, lo) = mulhilo(M, c), Weyl key bumps.  Counter-based: every (key,
// counter) pair is its own stream, no state in memory.
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
    constexpr unsigned M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const unsigned hi0 = __umulhi(M0, c.x), lo0 = M0 * c.x;
        const unsigned hi1 = __umulhi(M1, c.z), lo1 = M1 * c.z;
        c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
        k.x += W0;
        k.y += W1;
    }
    return c;
}
// uniform in (0, 1) from 32 random bits: (2 (x >> 9) + 1) * 2^-24, exactly
// representable in fp32, in [2^-24, 1 - 2^-24]
__device__ __forceinline__ float pt_u01(unsigned x) {
    return ((float)(x >> 9) * 2.0f + 1.0f) * 5.9604644775390625e-08f;
}

// fp32 id read back from an obs row: C cast truncates toward zero, then clamp
__device__ __forceinline__ int pt_id_clamp(float v, int hi) {
    int i = (int)v;
    return i < 0 ? 0 : (i > hi ? hi : i);
}

// wave64 reductions (DPP/permute via __shfl_xor)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// row pointer of obs row n, optionally through an int32 row-index list
__device__ __forceinline__ const float* obs_row(const float* obs, const int32_t* idx,
                                                long stride, int n) {
    long r = idx ? (long)idx[n] : (long)n;
    return obs + r * stride;
}

// ---------------------------------------------------------------- GEMM API
// C[M,N] = epi( sum_k A(m,k) B(k,n) ),
//   A(m,k) = a_t ? A[k*lda+m] : A[m*lda+k];  B(k,n) = b_t ? B[k*ldb+n] : B[n*ldb+k]
enum PtEpi {
    EPI_STORE = 0,      // C = acc
    EPI_BIAS = 1,       // C = acc + bias[n]
    EPI_BIAS_GELU = 2,  // C = acc + bias[n]; C2 = gelu(C)
    EPI_BIAS_RESID = 3, // C = acc + bias[n] + R[m*ldr+n]
    EPI_GELU_BWD = 4,   // C = acc * gelu'(R[m*ldr+n])
    EPI_ACCUM = 5,      // C += acc
    // the model's form of a GELU layer: the forward keeps gelu'(z) instead
    // of z (the backward needs nothing else of z), so the backward epilogue
    // is one multiply
    EPI_BIAS_GELU_D = 6,  // z = acc + bias[n]; C = gelu'(z); C2 = gelu(z)
    EPI_MUL = 7,          // C = acc * R[m*ldr+n]
    EPI_AXPBY = 8,        // C = alpha * acc + beta * R[m*ldr+n] (alpha, beta in GemmArgs)
};

struct GemmArgs {
    int M, N, K;
    const float* A; long lda;
    const float* B; long ldb;
    float* C; long ldc;
    const float* bias;
    const float* R; long ldr;
    float* C2; long ldc2;
    int a_t, b_t, epi;
    // optional, a_t == 1 with the STORE epilogue only: dbias[m] = sum_k A[k][m]
    // (the bias gradient of a weight-gradient product dW = dY^T X)
    float* dbias;
    // 0: fp32 products (v_mfma_f32_16x16x4_f32); 1: operands rounded to bf16
    // on the way into LDS, fp32 accumulation (v_mfma_f32_16x16x32_bf16)
    int prec;
    // bf16 storage: bs = A and B hold bf16 (k-contiguous both: C = epi(A B^T),
    // K, lda, ldb multiples of 8; or both transposed: the weight gradient
    // dW = A^T B, M, N, lda, ldb multiples of 8); obf = C (and C2) hold bf16,
    // as does R for EPI_MUL.  Pointers stay float* and are reinterpreted.
    int bs, obf;
    // set by pt_gemm: a launch covers logical tiles [tile0, tile0 + ntiles)
    // (ntiles 0 = all); tail_part: split-K partials of those tiles go to a
    // tile-local workspace [split][tile][128 x 128]
    int tile0, ntiles, tail_part;
    // set by pt_gemm: fp32 products through the LDS-DMA kernel
    int dma;
    // optional device row counts (stream-ordered compact layouts): the
    // product covers min(*Mdev, M) rows of A / C and min(*Kdev, K) of the
    // reduction; launches are sized for M and K
    const int* Mdev;
    const int* Kdev;
    // EPI_AXPBY scalars
    float alpha, beta;
    // set by pt_gemm for a weight gradient (A transposed) with a device
    // reduction count on the fp32 LDS-DMA kernel: the CU count, and the
    // launch's K splits follow pt_wgrad_splits of the device count (capped
    // at the launched splits; later splits return), which workgroup (0, 0, 0)
    // writes as an int after the partials for the reduce (0 = splits fixed
    // by the host)
    int wsplit;
};

// K splits of a weight gradient (A transposed, reduction over K rows) of
// `tiles` output tiles on `cu` CUs at k-step bk: a whole number of workgroups
// per CU, K / 128 rounded to the nearest multiple of the CU count (down: the
// multiple below; 1 .. 4 per CU), with chunks of at least 16 k-steps (4 below
// K = 64 bk).  Host and device share it, so a device reduction count splits
// as the same count given on the host would.
__host__ __device__ inline int pt_wgrad_splits(int K, int tiles, int cu, int bk, bool down = false) {
    if (K <= 0 || tiles <= 0) return 1;
    int per_cu = (K / 128 + (down ? 0 : cu / 2)) / cu;
    per_cu = per_cu < 1 ? 1 : per_cu > 4 ? 4 : per_cu;
    const int target = per_cu * cu;
    int splits = 1;
    if (tiles < target && K >= 2 * bk * 4) {
        splits = target / tiles;
        const int min_steps = K >= 4 * bk * 16 ? 16 : 4;
        const int max_splits = K / (bk * min_steps);
        if (splits > max_splits) splits = max_splits;
        if (splits < 1) splits = 1;
    }
    return splits;
}
// a split count's chunk of K, rounded up to the k-step, and the count that
// chunk gives (<= splits; every split but the last a full chunk)
__host__ __device__ inline int pt_split_chunks(int K, int splits, int bk, int* kc) {
    *kc = K > 0 ? K : bk;
    if (splits <= 1 || K <= 0) return 1;
    *kc = ((K + splits - 1) / splits + bk - 1) / bk * bk;
    return (K + *kc - 1) / *kc;
}

// Launch C = epi(A*B) on `stream`. Requirements: K % 4 == 0 when the operand
// is k-contiguous, M (N) % 4 == 0 when A (B) is m- (n-) contiguous, leading
// dims multiples of 4, 16 B-aligned bases.  Weight-gradient shapes
// (large K, small M*N) are split over K with a deterministic reduction.
int pt_gemm(const GemmArgs& g, float* splitk_ws, long splitk_ws_floats, hipStream_t s);
// C = A W^T + bias + R (N = 256; fp32 or, with g.bs, bf16 operands) and, in
// the same launch, y = LayerNorm(C) with its mean / rstd (eps 1e-5; ybf: y in
// bf16); pt_gemm_resid_ln_fits says whether g fits
bool pt_gemm_resid_ln_fits(const GemmArgs& g);
int pt_gemm_resid_ln(const GemmArgs& g, const float* lnw, const float* lnb, float* y, long ldy, float* mean,
                     float* rstd, hipStream_t s, int ybf = 0);
// the bf16 dX product dy = dY W (N = 256, W^T copy k-contiguous) with the
// LayerNorm backward of dy in the same launch: dx = LN'(dy) (+ dres), its
// bf16 copy dxh (nullable), dw / db overwritten; pt_dx_lnbwd_fits says
// whether g fits
bool pt_dx_lnbwd_fits(const GemmArgs& g);
int pt_dx_lnbwd(const GemmArgs& g, const float* x, const float* w, const float* mean, const float* rstd,
                const float* dres, float* dx, float* dxh, float* dw, float* db, float* ws, long ws_floats,
                hipStream_t s);

// One product of a grouped launch (pt_gemm_grouped): all products of a
// launch share the operand layout (a_t, b_t) and epilogue, and must meet the
// LDS-DMA tile rules (16 B-aligned operands, leading dimensions multiples of
// 4, K a multiple of 16 for k-contiguous operands).  Split-K products write
// `splits` partials of M x ldc at g.C (part_stride apart) and
// pt_grouped_reduce sums them into out.
struct GroupedGemm {
    GemmArgs g;
    int k_chunk, splits, tiles, first;   // first = the product's first work item
    long part_stride;
    float* out;
};
// items = sum of tiles * splits; item_group[w] = product of work item w
// flops: the launch's products (2 M N K summed; for launch timing only)
int pt_gemm_grouped(const GroupedGemm* d_groups, const int* d_item_group, int items, int a_t, int b_t, int epi,
                    int partial, double flops, hipStream_t s);
int pt_grouped_reduce(const GroupedGemm* d_groups, const int* d_chunk_group, const int* d_chunk_first, int chunks,
                      hipStream_t s);

// Linear helpers on row-major activations X (rows, in) and W (out, in)
int pt_linear_fwd(const float* X, const float* W, const float* b, float* Y, int rows,
                  int in, int out, int epi, const float* R, float* Y2, hipStream_t s);
// dX = dY W  (epi: EPI_STORE, EPI_ACCUM or EPI_GELU_BWD with R = pre-activation)
int pt_linear_dx(const float* dY, const float* W, float* dX, int rows, int in, int out,
                 int epi, const float* R, hipStream_t s);
// dW = dY^T X (overwrite), db = colsum(dY) (overwrite, may be NULL)
int pt_linear_dw(const float* dY, const float* X, float* dW, float* db, int rows, int in,
                 int out, float* ws, long ws_floats, hipStream_t s);

// deterministic column sums: out[n] = sum_m X[m*ldx + n], m < M
int pt_colsum(const float* X, long ldx, int M, int N, float* out, float* ws, long ws_floats,
              hipStream_t s);
// same, columns n < split to out_lo[n], the rest to out_hi[n - split]
int pt_colsum2(const float* X, long ldx, int M, int N, int split, float* out_lo, float* out_hi,
               float* ws, long ws_floats, hipStream_t s);
