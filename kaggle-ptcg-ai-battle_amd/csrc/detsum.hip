// Order-independent scatter-adds for the embedding-table gradients.
//
// The reference scatters every row's gradient into the shared tables (card,
// attack, zone, owner, option type, select type, context rows) with fp32
// atomicAdd (native/model/ptcg_model2.cu k_*_bwd, ptcg_kernels.cuh:84-96), so
// the sums depend on the order the atomics land in.  Here a scatter site
// (the kernels that add into a set of tables at one point of the backward)
// accumulates in 64-bit fixed point instead: integer addition is
// associative, so the result does not depend on the order and two identical
// backward calls give bit-identical gradients.
//
// Per site:
//   1. det_absmax_kernel: max |g| over each source slice (the gradient
//      columns the site scatters), DET_PART per-block partial maxima per
//      source (no atomics), 128-bit loads where the slice is aligned;
//   2. det_scale_kernel: per table t, scale_t = 2^(61 - e) with
//      2^e > count_t * max|g| (count_t bounds how many contributions one
//      table element can receive), so no partial sum can overflow 2^62;
//   3. the scatter kernels add rint(a * scale_t) for each fp32 partial sum a
//      of their id cache (detsum_add);
//   4. det_finish_kernel: table += acc * 2^-scale exponent, and the
//      accumulator is zeroed for the next site.
// A non-finite gradient makes its table NaN (the reference's atomics would
// spread it into the sums as well).  Resolution: 2^-61 of the largest sum a
// table element could reach, far below fp32's 2^-24 of the element itself
// unless the element is ~2^-37 of that bound.
#include "model.h"

namespace {

constexpr int DT_TB = 256;

__device__ __forceinline__ unsigned abits(float v) { return __float_as_uint(v) & 0x7fffffffu; }

// grid (DET_PART, nsrc): block b of source si takes elements b, b + DET_PART * DT_TB, ...
// of the source's rows x width slice; 128-bit loads where the slice allows
// (vec[si]: 16 B aligned rows, width and column a multiple of 4)
__global__ __launch_bounds__(DT_TB) void det_absmax_kernel(DetSite S, float* __restrict__ part) {
    const int si = blockIdx.y;
    const long rows = S.srows_dev[si] ? min((long)*S.srows_dev[si], S.srows[si]) : S.srows[si];
    const int w = S.swidth[si];
    const float* base = S.sp[si] + S.scol[si];
    const long ld = S.sld[si];
    unsigned mb = 0u;   // |v| as bits: integer order = float order, NaN above inf
    if (S.svec[si]) {
        const unsigned w4 = (unsigned)w >> 2;
        const unsigned total = (unsigned)rows * w4;   // host: rows * width < 2^31
        for (unsigned i = blockIdx.x * DT_TB + threadIdx.x; i < total; i += DET_PART * DT_TB) {
            const unsigned r = i / w4, c = i - r * w4;
            const float4 v = *reinterpret_cast<const float4*>(base + (long)r * ld + 4 * c);
            mb = max(mb, max(max(abits(v.x), abits(v.y)), max(abits(v.z), abits(v.w))));
        }
    } else {
        const unsigned total = (unsigned)rows * (unsigned)w;
        for (unsigned i = blockIdx.x * DT_TB + threadIdx.x; i < total; i += DET_PART * DT_TB) {
            const unsigned r = i / (unsigned)w, c = i - r * (unsigned)w;
            mb = max(mb, abits(base[(long)r * ld + c]));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mb = max(mb, (unsigned)__shfl_xor((int)mb, o, 64));
    __shared__ unsigned red[DT_TB / 64];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mb;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned m = red[0];
        for (int k = 1; k < DT_TB / 64; ++k) m = max(m, red[k]);
        part[si * DET_PART + blockIdx.x] = __uint_as_float(m);
    }
}

// one wave per table: max over its sources' partials, then the scale
__global__ __launch_bounds__(64 * DET_MAX_TAB) void det_scale_kernel(DetSite S, const float* __restrict__ part,
                                                                    double* __restrict__ scale) {
    const int t = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (t >= S.ntab) return;
    unsigned mb = 0u;
    for (int si = 0; si < S.nsrc; ++si) {
        if (S.stab[si] != t) continue;
        for (int k = lane; k < DET_PART; k += 64) mb = max(mb, __float_as_uint(part[si * DET_PART + k]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mb = max(mb, (unsigned)__shfl_xor((int)mb, o, 64));
    if (lane != 0) return;
    double sc;
    if (mb >= 0x7f800000u) {
        sc = -1.0;   // non-finite gradient: the table becomes NaN
    } else if (mb == 0u) {
        sc = 1.0;    // nothing to add
    } else {
        int e;
        (void)frexp((double)__uint_as_float(mb) * S.count[t], &e);   // bound < 2^e
        sc = ldexp(1.0, 61 - e);
    }
    scale[t] = sc;
}

__global__ __launch_bounds__(DT_TB) void det_finish_kernel(DetSite S, unsigned long long* __restrict__ acc,
                                                           const double* __restrict__ scale) {
    const int t = blockIdx.y;
    const double sc = scale[t];
    unsigned long long* a = acc + S.acc_off[t];
    float* tab = S.tab[t];
    for (long i = (long)blockIdx.x * DT_TB + threadIdx.x; i < S.tab_n[t]; i += (long)gridDim.x * DT_TB) {
        const unsigned long long v = a[i];
        a[i] = 0ull;
        if (sc < 0.0) tab[i] = __int_as_float(0x7fc00000);
        else if (v) tab[i] += (float)((double)(long long)v / sc);
    }
}

}  // namespace

int pt_det_prepare(const DetCtx& d, const DetSite& S, hipStream_t s) {
    PT_REQUIRE(d.acc && d.part && d.scale, "det: accumulators not allocated (training registration)");
    PT_REQUIRE(S.ntab >= 1 && S.ntab <= DET_MAX_TAB && S.nsrc >= 1 && S.nsrc <= DET_MAX_SRC,
               "det: %d tables / %d sources", S.ntab, S.nsrc);
    for (int t = 0; t < S.ntab; ++t)
        PT_REQUIRE(S.acc_off[t] >= 0 && S.acc_off[t] + S.tab_n[t] <= d.acc_len,
                   "det: table %d needs accumulator [%ld, %ld) of %ld", t, S.acc_off[t], S.acc_off[t] + S.tab_n[t],
                   d.acc_len);
    DetSite V = S;
    for (int i = 0; i < S.nsrc; ++i) {
        PT_REQUIRE(S.stab[i] >= 0 && S.stab[i] < S.ntab, "det: source %d maps to table %d", i, S.stab[i]);
        PT_REQUIRE(S.srows[i] * S.swidth[i] < (1L << 31), "det: source %d of %ld x %d elements", i, S.srows[i],
                   S.swidth[i]);
        V.svec[i] = (((uintptr_t)S.sp[i] & 15) == 0 && S.sld[i] % 4 == 0 && S.scol[i] % 4 == 0 &&
                     S.swidth[i] % 4 == 0) ? 1 : 0;
    }
    hipLaunchKernelGGL(det_absmax_kernel, dim3(DET_PART, V.nsrc), dim3(DT_TB), 0, s, V, d.part);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(det_scale_kernel, dim3(1), dim3(64 * DET_MAX_TAB), 0, s, V, (const float*)d.part, d.scale);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

int pt_det_finish(const DetCtx& d, const DetSite& S, hipStream_t s) {
    long mx = 0;
    for (int t = 0; t < S.ntab; ++t) mx = S.tab_n[t] > mx ? S.tab_n[t] : mx;
    const int gx = (int)std::min<long>(pt_cdiv(mx, DT_TB), 1024);
    hipLaunchKernelGGL(det_finish_kernel, dim3(gx, S.ntab), dim3(DT_TB), 0, s, S, d.acc, (const double*)d.scale);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

DetSink pt_det_sink(const DetCtx& d, const DetSite& S, int t, long ld) {
    return DetSink{d.acc + S.acc_off[t], d.scale + t, ld};
}
