// bf16 copies for the mixed-precision variant (bf16 activations in HBM, the
// reference's precision_t = bf16 build, native/src/kernels.cu:25-30).
//
// pt_bf16_weights: the trunk blocks' weight matrices W (out, in), fp32
// masters, to bf16 W (out, in) for the forward products C = X W^T and bf16
// W^T (in, out) for the backward's dX = dY W, so that both read their weight
// operand k-contiguous.  One launch over every matrix: 32 x 32 tiles, a
// workgroup per tile, the transpose through LDS (both stores coalesced).
// Run at the start of each bf16 forward, so the copies always follow the
// masters (after an optimizer step or a weight load) and the step stays
// graph-capturable; ~25 MB of traffic for the CORE trunk.
//
// pt_to_bf16: an fp32 array to bf16 (round to nearest even).
#include "model.h"

namespace {

constexpr int WT = 32;

__global__ __launch_bounds__(256) void bf16_weights_kernel(BfWeightSet ws) {
    __shared__ float tile[WT][WT + 1];
    int mi = 0;
    while (mi + 1 < ws.n && (int)blockIdx.x >= ws.m[mi + 1].tile0) ++mi;
    const BfWeight& w = ws.m[mi];
    const int t = blockIdx.x - w.tile0;
    const int tc = (w.cols + WT - 1) / WT;
    const int r0 = (t / tc) * WT, c0 = (t % tc) * WT;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8
#pragma unroll
    for (int k = 0; k < WT; k += 8) {
        const int r = r0 + ty + k, c = c0 + tx;
        float v = 0.f;
        if (r < w.rows && c < w.cols) {
            v = w.src[(long)r * w.cols + c];
            w.dst[(long)r * w.cols + c] = (__bf16)v;
        }
        tile[ty + k][tx] = v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < WT; k += 8) {
        const int c = c0 + ty + k, r = r0 + tx;   // element (r, c) -> dstT[c][r]
        if (r < w.rows && c < w.cols) w.dstT[(long)c * w.rows + r] = (__bf16)tile[tx][ty + k];
    }
}

__global__ __launch_bounds__(256) void to_bf16_kernel(const float* __restrict__ src, __bf16* __restrict__ dst,
                                                      long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = (__bf16)src[i];
}

}  // namespace

int pt_bf16_weights(BfWeightSet& ws, hipStream_t s) {
    PT_REQUIRE(ws.n >= 1 && ws.n <= BF_MAX_W, "bf16 weights: %d matrices", ws.n);
    int tiles = 0;
    for (int i = 0; i < ws.n; ++i) {
        PT_REQUIRE(ws.m[i].src && ws.m[i].dst && ws.m[i].dstT && ws.m[i].rows > 0 && ws.m[i].cols > 0,
                   "bf16 weights: matrix %d incomplete", i);
        ws.m[i].tile0 = tiles;
        tiles += pt_cdiv(ws.m[i].rows, WT) * pt_cdiv(ws.m[i].cols, WT);
    }
    hipLaunchKernelGGL(bf16_weights_kernel, dim3(tiles), dim3(256), 0, s, ws);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

int pt_to_bf16(const float* src, float* dst, long n, hipStream_t s) {
    if (n <= 0) return PTCG_OK;
    hipLaunchKernelGGL(to_bf16_kernel, dim3(pt_cdiv(n, 256)), dim3(256), 0, s, src, reinterpret_cast<__bf16*>(dst),
                       n);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
