// Compact trunk layout: only the rows that can reach an output are computed.
//
// The reference runs every one of the l_tok + 1 trunk positions of every
// sample (ptcg_model3.cu:246-300) and masks padded tokens out of the keys
// (keep = zone > 0, ptcg_model.cu:360-367).  A padded position is never a
// key, so it influences no other row; its own trunk output reaches the heads
// only when an option pointer selects it (ptcg_model.cu:405-411).  The rows
// that matter per sample are therefore READOUT, the valid tokens and the
// pointer targets ("active"); every other row's output is unused and its
// gradient is zero, so dropping those rows changes no result.  Sample n's
// active rows are stored contiguously, READOUT first then positions in
// order, at rows [coff[n], coff[n+1]); GEMMs, LayerNorms and attention run
// over coff[N] rows (read from the device, launches sized for N * l_seq).
#include "model.h"

namespace {

// one workgroup per sample: act[pos] = 1 for READOUT, valid tokens and the
// targets of any option pointer (legal or not: every slot's score is output)
__global__ void compact_count_kernel(GatherCtx c, int* __restrict__ act, int* __restrict__ cnt) {
    const int n = blockIdx.x, Ls = c.dx.l_seq, Lt = c.dm.l_tok;
    const float* row = obs_row(c.obs, c.idx, c.stride, n);
    int* a = act + (long)n * Ls;
    for (int p = threadIdx.x; p < Ls; p += blockDim.x)
        a[p] = p == 0 ? 1 : (row[c.off.tok_int + (long)(p - 1) * c.dm.tok_int + 1] > 0.f ? 1 : 0);
    __syncthreads();
    for (int j = threadIdx.x; j < c.dm.n_opt; j += blockDim.x) {
        const float* oi = row + c.off.opt_int + (long)j * c.dm.opt_int;
        const int p1 = (int)oi[1], p2 = (int)oi[2];
        if (p1 > 0 && p1 <= Lt) a[p1] = 1;   // benign race: every writer stores 1
        if (p2 > 0 && p2 <= Lt) a[p2] = 1;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        int s = 0;
        for (int p = threadIdx.x; p < Ls; p += 64) s += a[p];
        s = (int)wave_sum((float)s);   // <= 257, exact
        if (threadIdx.x == 0) cnt[n] = s;
    }
}

// exclusive prefix sum of cnt -> coff[0..N] (one workgroup, fixed order)
__global__ void compact_scan_kernel(const int* __restrict__ cnt, int N, int* __restrict__ coff) {
    __shared__ int part[256];
    const int t = threadIdx.x;
    const int per = (N + 255) / 256;
    const int b = t * per, e = min(N, b + per);
    int s = 0;
    for (int i = b; i < e; ++i) s += cnt[i];
    part[t] = s;
    __syncthreads();
    if (t == 0) {
        int acc = 0;
        for (int i = 0; i < 256; ++i) {
            const int v = part[i];
            part[i] = acc;
            acc += v;
        }
        coff[N] = acc;
    }
    __syncthreads();
    int acc = part[t];
    for (int i = b; i < e; ++i) {
        coff[i] = acc;
        acc += cnt[i];
    }
}

// one wave per sample: rank the active positions in order
__global__ void compact_fill_kernel(GatherCtx c, const int* __restrict__ act, const int* __restrict__ coff,
                                    int* __restrict__ rowmap, int* __restrict__ rsam, int* __restrict__ rpos) {
    const int n = blockIdx.x, Ls = c.dx.l_seq, lane = threadIdx.x;
    const int* a = act + (long)n * Ls;
    int base = coff[n];
    for (int p0 = 0; p0 < Ls; p0 += 64) {
        const int p = p0 + lane;
        const int on = p < Ls ? a[p] : 0;
        const unsigned long long bal = __ballot(on);
        const int rank = __popcll(bal & ((1ull << lane) - 1ull));
        if (p < Ls) {
            const int r = on ? base + rank : -1;
            rowmap[(long)n * Ls + p] = r;
            if (on) {
                rsam[r] = n;
                rpos[r] = p;
            }
        }
        base += __popcll(bal);
    }
}

// One wave per sample: the legal options (mask != 0) of sample n, or all of
// them when none is legal.  A masked option's score enters the loss only as
// the constant -1e4 and gets exactly zero gradient whenever some option is
// legal, so only these rows need the option scorer in training.
__device__ __forceinline__ bool opt_on(const float* mk, int j, bool none) { return none || mk[j] != 0.f; }
__global__ void opt_count_kernel(GatherCtx c, int* __restrict__ cnt) {
    const int n = blockIdx.x, NO = c.dm.n_opt, lane = threadIdx.x;
    const float* mk = obs_row(c.obs, c.idx, c.stride, n) + c.off.opt_mask;
    int legal = 0;
    for (int j0 = 0; j0 < NO; j0 += 64) {
        const int j = j0 + lane;
        legal += __popcll(__ballot(j < NO && mk[j] != 0.f));
    }
    if (lane == 0) cnt[n] = legal > 0 ? legal : NO;
}
__global__ void opt_fill_kernel(GatherCtx c, const int* __restrict__ ooff, int* __restrict__ orow) {
    const int n = blockIdx.x, NO = c.dm.n_opt, lane = threadIdx.x;
    const float* mk = obs_row(c.obs, c.idx, c.stride, n) + c.off.opt_mask;
    int legal = 0;
    for (int j0 = 0; j0 < NO; j0 += 64) legal += __popcll(__ballot(j0 + lane < NO && mk[j0 + lane] != 0.f));
    const bool none = legal == 0;
    int base = ooff[n];
    for (int j0 = 0; j0 < NO; j0 += 64) {
        const int j = j0 + lane;
        const bool on = j < NO && opt_on(mk, j, none);
        const unsigned long long bal = __ballot(on);
        if (on) orow[base + __popcll(bal & ((1ull << lane) - 1ull))] = n * NO + j;
        base += __popcll(bal);
    }
}

__global__ void gather_rows_kernel(const float* __restrict__ src, long ld, const int* __restrict__ coff, int N,
                                   int D, float* __restrict__ dst) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)N * D) return;
    const int n = (int)(i / D), d = (int)(i % D);
    dst[i] = src[(long)coff[n] * ld + d];
}

}  // namespace

int pt_compact_map(const GatherCtx& c, int* act, int* cnt, int* coff, int* rowmap, int* rsam, int* rpos,
                   hipStream_t s) {
    PT_REQUIRE(c.dx.l_seq <= 4096, "compact map: l_seq %d too long", c.dx.l_seq);
    hipLaunchKernelGGL(compact_count_kernel, dim3(c.N), dim3(128), 0, s, c, act, cnt);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(compact_scan_kernel, dim3(1), dim3(256), 0, s, cnt, c.N, coff);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(compact_fill_kernel, dim3(c.N), dim3(64), 0, s, c, act, coff, rowmap, rsam, rpos);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

int pt_opt_map(const GatherCtx& c, int* cnt, int* ooff, int* orow, hipStream_t s) {
    hipLaunchKernelGGL(opt_count_kernel, dim3(c.N), dim3(64), 0, s, c, cnt);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(compact_scan_kernel, dim3(1), dim3(256), 0, s, cnt, c.N, ooff);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(opt_fill_kernel, dim3(c.N), dim3(64), 0, s, c, ooff, orow);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

int pt_gather_rows(const float* src, long ld, const int* coff, int N, int D, float* dst, hipStream_t s) {
    hipLaunchKernelGGL(gather_rows_kernel, dim3(pt_cdiv((long)N * D, 256)), dim3(256), 0, s, src, ld, coff, N, D,
                       dst);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
