// LayerNorm forward / backward (eps 1e-5, biased variance: torch nn.LayerNorm).
//
// Replaces pt_ln_fwd / pt_ln_bwd (native/model/ptcg_kernels.cuh:132-218):
// one wave64 per row with the row held in registers as float4s (the
// reference uses one 128-thread block per row), two-pass mean/variance.
// Backward writes dx (optionally adding a residual gradient in the same
// pass) and per-workgroup dW/dB partials (512 workgroups stride over the
// rows) that a two-level column sum folds in fixed order — deterministic,
// where the reference issues one atomicAdd per element per row into 2*D
// addresses.
#include "common.h"

namespace {

constexpr int LN_BWD_BLOCKS = 512;   // partial rows of dW/dB (grid-stride over rows)

template <int VPL>
__global__ __launch_bounds__(256) void ln_fwd_kernel(const float* __restrict__ x, long ldx,
        const float* __restrict__ w, const float* __restrict__ b, float* __restrict__ y, long ldy,
        float* __restrict__ mean, float* __restrict__ rstd, int rows, int D,
        const int* __restrict__ rows_dev) {
    if (rows_dev) rows = min(rows, *rows_dev);   // device row count (compact layouts)
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + (long)row * ldx;
    float4 v[VPL];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
        const int col = (lane + 64 * c) * 4;
        v[c] = col < D ? *reinterpret_cast<const float4*>(xr + col) : make_float4(0.f, 0.f, 0.f, 0.f);
        s += (v[c].x + v[c].y) + (v[c].z + v[c].w);
    }
    const float mu = wave_sum(s) / (float)D;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
        const int col = (lane + 64 * c) * 4;
        if (col < D) {
            float a = v[c].x - mu, bb = v[c].y - mu, cc = v[c].z - mu, dd = v[c].w - mu;
            q += (a * a + bb * bb) + (cc * cc + dd * dd);
        }
    }
    const float var = wave_sum(q) / (float)D;
    const float rs = 1.0f / sqrtf(var + 1e-5f);
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = rs;
    }
    float* yr = y + (long)row * ldy;
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
        const int col = (lane + 64 * c) * 4;
        if (col < D) {
            const float4 ww = *reinterpret_cast<const float4*>(w + col);
            const float4 bb = *reinterpret_cast<const float4*>(b + col);
            float4 o;
            o.x = (v[c].x - mu) * rs * ww.x + bb.x;
            o.y = (v[c].y - mu) * rs * ww.y + bb.y;
            o.z = (v[c].z - mu) * rs * ww.z + bb.z;
            o.w = (v[c].w - mu) * rs * ww.w + bb.w;
            *reinterpret_cast<float4*>(yr + col) = o;
        }
    }
}

// dx = rs*(g - mean(g) - xh*mean(g*xh)) [+ dres], g = dy*w, xh = (x-mu)*rs.
// part[blk][0..D) = sum dy*xh, part[blk][D..2D) = sum dy over the block's rows.
template <int VPL>
__global__ __launch_bounds__(256) void ln_bwd_kernel(const float* __restrict__ dy, long lddy,
        const float* __restrict__ x, long ldx, const float* __restrict__ w,
        const float* __restrict__ mean, const float* __restrict__ rstd,
        const float* __restrict__ dres, long ldres, float* __restrict__ dx, long lddx,
        float* __restrict__ part, int rows, int D,
        const int* __restrict__ rows_dev) {
    if (rows_dev) rows = min(rows, *rows_dev);   // device row count (compact layouts)
    __shared__ float4 sh_w[4][VPL * 64];
    __shared__ float4 sh_b[4][VPL * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float4 aw[VPL], ab[VPL];
    float4 wv[VPL];
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
        aw[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        ab[c] = aw[c];
        const int col = (lane + 64 * c) * 4;
        wv[c] = col < D ? *reinterpret_cast<const float4*>(w + col) : aw[c];
    }
    for (int row = blockIdx.x * 4 + wave; row < rows; row += gridDim.x * 4) {
        const float mu = mean[row], rs = rstd[row];
        const float* xr = x + (long)row * ldx;
        const float* dyr = dy + (long)row * lddy;
        float4 xh[VPL], g[VPL], d[VPL];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int c = 0; c < VPL; ++c) {
            const int col = (lane + 64 * c) * 4;
            if (col < D) {
                float4 xv = *reinterpret_cast<const float4*>(xr + col);
                d[c] = *reinterpret_cast<const float4*>(dyr + col);
                xh[c] = make_float4((xv.x - mu) * rs, (xv.y - mu) * rs, (xv.z - mu) * rs, (xv.w - mu) * rs);
                g[c] = make_float4(d[c].x * wv[c].x, d[c].y * wv[c].y, d[c].z * wv[c].z, d[c].w * wv[c].w);
                s1 += (g[c].x + g[c].y) + (g[c].z + g[c].w);
                s2 += (g[c].x * xh[c].x + g[c].y * xh[c].y) + (g[c].z * xh[c].z + g[c].w * xh[c].w);
                aw[c].x += d[c].x * xh[c].x; aw[c].y += d[c].y * xh[c].y;
                aw[c].z += d[c].z * xh[c].z; aw[c].w += d[c].w * xh[c].w;
                ab[c].x += d[c].x; ab[c].y += d[c].y; ab[c].z += d[c].z; ab[c].w += d[c].w;
            }
        }
        const float m1 = wave_sum(s1) / (float)D;
        const float m2 = wave_sum(s2) / (float)D;
        float* dxr = dx + (long)row * lddx;
        const float* dr = dres ? dres + (long)row * ldres : nullptr;
#pragma unroll
        for (int c = 0; c < VPL; ++c) {
            const int col = (lane + 64 * c) * 4;
            if (col < D) {
                float4 o;
                o.x = (g[c].x - m1 - xh[c].x * m2) * rs;
                o.y = (g[c].y - m1 - xh[c].y * m2) * rs;
                o.z = (g[c].z - m1 - xh[c].z * m2) * rs;
                o.w = (g[c].w - m1 - xh[c].w * m2) * rs;
                if (dr) {
                    const float4 rv = *reinterpret_cast<const float4*>(dr + col);
                    o.x += rv.x; o.y += rv.y; o.z += rv.z; o.w += rv.w;
                }
                *reinterpret_cast<float4*>(dxr + col) = o;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
        sh_w[wave][lane + 64 * c] = aw[c];
        sh_b[wave][lane + 64 * c] = ab[c];
    }
    __syncthreads();
    // wave 0 folds the 4 waves in fixed order and writes this block's partial
    if (wave == 0) {
        float* pw = part + (long)blockIdx.x * 2 * D;
#pragma unroll
        for (int c = 0; c < VPL; ++c) {
            const int col = (lane + 64 * c) * 4;
            if (col < D) {
                float4 sw = sh_w[0][lane + 64 * c], sb = sh_b[0][lane + 64 * c];
                for (int k = 1; k < 4; ++k) {
                    float4 a = sh_w[k][lane + 64 * c], bq = sh_b[k][lane + 64 * c];
                    sw.x += a.x; sw.y += a.y; sw.z += a.z; sw.w += a.w;
                    sb.x += bq.x; sb.y += bq.y; sb.z += bq.z; sb.w += bq.w;
                }
                *reinterpret_cast<float4*>(pw + col) = sw;
                *reinterpret_cast<float4*>(pw + D + col) = sb;
            }
        }
    }
}

// Scalar variants for widths that are not multiples of 4 (the reference's
// 634-wide card LayerNorm): element col = lane + 64c, up to 16 per lane.
constexpr int LN_SC = 16;

__global__ __launch_bounds__(256) void ln_fwd_scalar_kernel(const float* __restrict__ x, long ldx,
        const float* __restrict__ w, const float* __restrict__ b, float* __restrict__ y, long ldy,
        float* __restrict__ mean, float* __restrict__ rstd, int rows, int D,
        const int* __restrict__ rows_dev) {
    if (rows_dev) rows = min(rows, *rows_dev);   // device row count (compact layouts)
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + (long)row * ldx;
    float v[LN_SC];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < LN_SC; ++c) {
        const int col = lane + 64 * c;
        v[c] = col < D ? xr[col] : 0.f;
        s += v[c];
    }
    const float mu = wave_sum(s) / (float)D;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < LN_SC; ++c)
        if (lane + 64 * c < D) q += (v[c] - mu) * (v[c] - mu);
    const float rs = 1.0f / sqrtf(wave_sum(q) / (float)D + 1e-5f);
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = rs;
    }
    float* yr = y + (long)row * ldy;
#pragma unroll
    for (int c = 0; c < LN_SC; ++c) {
        const int col = lane + 64 * c;
        if (col < D) yr[col] = (v[c] - mu) * rs * w[col] + b[col];
    }
}

__global__ __launch_bounds__(256) void ln_bwd_scalar_kernel(const float* __restrict__ dy, long lddy,
        const float* __restrict__ x, long ldx, const float* __restrict__ w,
        const float* __restrict__ mean, const float* __restrict__ rstd,
        const float* __restrict__ dres, long ldres, float* __restrict__ dx, long lddx,
        float* __restrict__ part, int rows, int D,
        const int* __restrict__ rows_dev) {
    if (rows_dev) rows = min(rows, *rows_dev);   // device row count (compact layouts)
    __shared__ float sh_w[4][LN_SC * 64];
    __shared__ float sh_b[4][LN_SC * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float aw[LN_SC], ab[LN_SC], wv[LN_SC];
#pragma unroll
    for (int c = 0; c < LN_SC; ++c) {
        aw[c] = 0.f;
        ab[c] = 0.f;
        const int col = lane + 64 * c;
        wv[c] = col < D ? w[col] : 0.f;
    }
    for (int row = blockIdx.x * 4 + wave; row < rows; row += gridDim.x * 4) {
        const float mu = mean[row], rs = rstd[row];
        const float* xr = x + (long)row * ldx;
        const float* dyr = dy + (long)row * lddy;
        float xh[LN_SC], g[LN_SC];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int c = 0; c < LN_SC; ++c) {
            const int col = lane + 64 * c;
            xh[c] = 0.f;
            g[c] = 0.f;
            if (col < D) {
                const float d = dyr[col];
                xh[c] = (xr[col] - mu) * rs;
                g[c] = d * wv[c];
                s1 += g[c];
                s2 += g[c] * xh[c];
                aw[c] += d * xh[c];
                ab[c] += d;
            }
        }
        const float m1 = wave_sum(s1) / (float)D;
        const float m2 = wave_sum(s2) / (float)D;
        float* dxr = dx + (long)row * lddx;
        const float* dr = dres ? dres + (long)row * ldres : nullptr;
#pragma unroll
        for (int c = 0; c < LN_SC; ++c) {
            const int col = lane + 64 * c;
            if (col < D) dxr[col] = (g[c] - m1 - xh[c] * m2) * rs + (dr ? dr[col] : 0.f);
        }
    }
#pragma unroll
    for (int c = 0; c < LN_SC; ++c) {
        sh_w[wave][lane + 64 * c] = aw[c];
        sh_b[wave][lane + 64 * c] = ab[c];
    }
    __syncthreads();
    if (wave == 0) {
        float* pw = part + (long)blockIdx.x * 2 * D;
#pragma unroll
        for (int c = 0; c < LN_SC; ++c) {
            const int col = lane + 64 * c;
            if (col < D) {
                pw[col] = ((sh_w[0][col] + sh_w[1][col]) + sh_w[2][col]) + sh_w[3][col];
                pw[D + col] = ((sh_b[0][col] + sh_b[1][col]) + sh_b[2][col]) + sh_b[3][col];
            }
        }
    }
}

bool ln_vec_ok(const void* p, long ld, int D) { return D % 4 == 0 && ld % 4 == 0 && ((uintptr_t)p & 15) == 0; }

}  // namespace

int pt_ln_fwd(const float* x, long ldx, const float* w, const float* b, float* y, long ldy,
              float* mean, float* rstd, int rows, int D, hipStream_t s, const int* rows_dev) {
    PT_REQUIRE(D >= 1 && D <= 1024, "layernorm: D=%d unsupported", D);
    dim3 grid(pt_cdiv(rows, 4));
    if (!(ln_vec_ok(x, ldx, D) && ln_vec_ok(y, ldy, D) && ln_vec_ok(w, 0, D) && ln_vec_ok(b, 0, D)))
        hipLaunchKernelGGL(ln_fwd_scalar_kernel, grid, dim3(256), 0, s, x, ldx, w, b, y, ldy, mean, rstd, rows, D, rows_dev);
    else if (D <= 256)
        hipLaunchKernelGGL(ln_fwd_kernel<1>, grid, dim3(256), 0, s, x, ldx, w, b, y, ldy, mean, rstd, rows, D, rows_dev);
    else if (D <= 512)
        hipLaunchKernelGGL(ln_fwd_kernel<2>, grid, dim3(256), 0, s, x, ldx, w, b, y, ldy, mean, rstd, rows, D, rows_dev);
    else
        hipLaunchKernelGGL(ln_fwd_kernel<4>, grid, dim3(256), 0, s, x, ldx, w, b, y, ldy, mean, rstd, rows, D, rows_dev);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

int pt_ln_bwd(const float* dy, long lddy, const float* x, long ldx, const float* w,
              const float* mean, const float* rstd, const float* dres, long ldres, float* dx,
              long lddx, float* dw, float* db, int rows, int D, float* ws, long ws_floats,
              hipStream_t s, const int* rows_dev) {
    PT_REQUIRE(D >= 1 && D <= 1024, "layernorm bwd: D=%d unsupported", D);
    int blocks = pt_cdiv(rows, 4);
    if (blocks > LN_BWD_BLOCKS) blocks = LN_BWD_BLOCKS;
    PT_REQUIRE(ws && (long)blocks * 2 * D * 2 <= ws_floats, "layernorm bwd: workspace too small");
    dim3 grid(blocks);
    const bool vec = ln_vec_ok(dy, lddy, D) && ln_vec_ok(x, ldx, D) && ln_vec_ok(w, 0, D) &&
                     ln_vec_ok(dx, lddx, D) && (dres == nullptr || ln_vec_ok(dres, ldres, D));
    if (!vec)
        hipLaunchKernelGGL(ln_bwd_scalar_kernel, grid, dim3(256), 0, s, dy, lddy, x, ldx, w, mean, rstd, dres, ldres, dx, lddx, ws, rows, D, rows_dev);
    else if (D <= 256)
        hipLaunchKernelGGL(ln_bwd_kernel<1>, grid, dim3(256), 0, s, dy, lddy, x, ldx, w, mean, rstd, dres, ldres, dx, lddx, ws, rows, D, rows_dev);
    else if (D <= 512)
        hipLaunchKernelGGL(ln_bwd_kernel<2>, grid, dim3(256), 0, s, dy, lddy, x, ldx, w, mean, rstd, dres, ldres, dx, lddx, ws, rows, D, rows_dev);
    else
        hipLaunchKernelGGL(ln_bwd_kernel<4>, grid, dim3(256), 0, s, dy, lddy, x, ldx, w, mean, rstd, dres, ldres, dx, lddx, ws, rows, D, rows_dev);
    PT_LAUNCH_CHECK();
    if (dw && db)
        return pt_colsum2(ws, 2 * D, blocks, 2 * D, D, dw, db, ws + (long)blocks * 2 * D,
                          ws_floats - (long)blocks * 2 * D, s);
    PT_REQUIRE(!dw && !db, "layernorm bwd: dw and db must both be given or both be NULL");
    return PTCG_OK;
}
