// LayerNorm forward / backward (eps 1e-5, biased variance: torch nn.LayerNorm).
//
// Replaces pt_ln_fwd / pt_ln_bwd (native/model/ptcg_kernels.cuh:132-218):
// one wave64 per row with the row held in registers as float4s (the
// reference uses one 128-thread block per row), two-pass mean/variance.
// Launch shapes (measured on 37.4k rows of d = 256): the forward runs one
// row per wave, 4 waves per workgroup (loading 2 or 4 rows per wave before
// reducing gained nothing); the backward runs 8-wave workgroups, 512 of them
// striding over the rows, one row per wave per iteration (the templates take
// rows per wave / per iteration for other shapes).
// Backward writes dx (optionally adding a residual gradient in the same
// pass) and per-workgroup dW/dB partials (LN_BWD_BLOCKS workgroups stride
// over the rows) that a two-level column sum folds in fixed order —
// deterministic, where the reference issues one atomicAdd per element per
// row into 2*D addresses.
#include "common.h"

namespace {

constexpr int LN_BWD_BLOCKS = 512;   // partial rows of dW/dB (grid-stride over rows)
constexpr int LN_FWD_RPW = 1;        // forward rows per wave, loaded together
constexpr int LN_BWD_WPB = 8;        // backward waves per workgroup (rows of d <= 256)
constexpr int LN_BWD_RPI = 1;        // backward rows per wave per iteration, loaded together

typedef __bf16 lnbf16x4 __attribute__((ext_vector_type(4)));
// four floats to bf16 (round to nearest even) at element i of a bf16 array
__device__ __forceinline__ void st_bf16x4(float* base, long i, float4 o) {
    *reinterpret_cast<lnbf16x4*>(reinterpret_cast<__bf16*>(base) + i) =
        lnbf16x4{(__bf16)o.x, (__bf16)o.y, (__bf16)o.z, (__bf16)o.w};
}

// rows blockIdx.x * 4 * RPW + wave + 4 r, r < RPW
// YB: y is stored in bf16 (the mixed-precision variant's GEMM operand)
template <int VPL, int RPW, bool YB = false>
__global__ __launch_bounds__(256) void ln_fwd_kernel(const float* __restrict__ x, long ldx,
        const float* __restrict__ w, const float* __restrict__ b, float* __restrict__ y, long ldy,
        float* __restrict__ mean, float* __restrict__ rstd, int rows, int D,
        const int* __restrict__ rows_dev) {
    if (rows_dev) rows = min(rows, *rows_dev);   // device row count (compact layouts)
    const int lane = threadIdx.x & 63;
    const int row0 = blockIdx.x * 4 * RPW + (threadIdx.x >> 6);
    if (row0 >= rows) return;
    float4 v[RPW][VPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row0 + 4 * r;
        const float* xr = x + (long)row * ldx;
#pragma unroll
        for (int c = 0; c < VPL; ++c) {
            const int col = (lane + 64 * c) * 4;
            v[r][c] = (row < rows && col < D) ? *reinterpret_cast<const float4*>(xr + col)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row0 + 4 * r;
        if (row >= rows) break;
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < VPL; ++c) s += (v[r][c].x + v[r][c].y) + (v[r][c].z + v[r][c].w);
        const float mu = wave_sum(s) / (float)D;
        float q = 0.f;
#pragma unroll
        for (int c = 0; c < VPL; ++c) {
            const int col = (lane + 64 * c) * 4;
            if (col < D) {
                float a = v[r][c].x - mu, bb = v[r][c].y - mu, cc = v[r][c].z - mu, dd = v[r][c].w - mu;
                q += (a * a + bb * bb) + (cc * cc + dd * dd);
            }
        }
        const float var = wave_sum(q) / (float)D;
        const float rs = 1.0f / sqrtf(var + 1e-5f);
        if (lane == 0) {
            mean[row] = mu;
            rstd[row] = rs;
        }
#pragma unroll
        for (int c = 0; c < VPL; ++c) {
            const int col = (lane + 64 * c) * 4;
            if (col < D) {
                const float4 ww = *reinterpret_cast<const float4*>(w + col);
                const float4 bb = *reinterpret_cast<const float4*>(b + col);
                float4 o;
                o.x = (v[r][c].x - mu) * rs * ww.x + bb.x;
                o.y = (v[r][c].y - mu) * rs * ww.y + bb.y;
                o.z = (v[r][c].z - mu) * rs * ww.z + bb.z;
                o.w = (v[r][c].w - mu) * rs * ww.w + bb.w;
                if (YB) st_bf16x4(y, (long)row * ldy + col, o);
                else *reinterpret_cast<float4*>(y + (long)row * ldy + col) = o;
            }
        }
    }
}

// dx = rs*(g - mean(g) - xh*mean(g*xh)) [+ dres], g = dy*w, xh = (x-mu)*rs.
// part[blk][0..D) = sum dy*xh, part[blk][D..2D) = sum dy over the block's rows.
// dxh (nullable): a bf16 copy of dx at the same leading dimension (the next
// products' operand in the mixed-precision variant).
// Wave w of workgroup b takes rows b*WPB + w + k*S (S = gridDim.x*WPB), RPI
// consecutive k at a time.
template <int VPL, int WPB, int RPI>
__global__ __launch_bounds__(64 * WPB) void ln_bwd_kernel(const float* __restrict__ dy, long lddy,
        const float* __restrict__ x, long ldx, const float* __restrict__ w,
        const float* __restrict__ mean, const float* __restrict__ rstd,
        const float* __restrict__ dres, long ldres, float* __restrict__ dx, long lddx,
        float* __restrict__ part, int rows, int D,
        const int* __restrict__ rows_dev, float* __restrict__ dxh) {
    if (rows_dev) rows = min(rows, *rows_dev);   // device row count (compact layouts)
    __shared__ float4 sh_w[WPB][VPL * 64];
    __shared__ float4 sh_b[WPB][VPL * 64];
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
    const int S = gridDim.x * WPB;
    for (int r0 = blockIdx.x * WPB + wave; r0 < rows; r0 += S * RPI) {
        float4 xv[RPI][VPL], d[RPI][VPL];
        float mu[RPI], rs[RPI];
#pragma unroll
        for (int k = 0; k < RPI; ++k) {
            const int row = r0 + k * S;
            const bool ok = row < rows;
            mu[k] = ok ? mean[row] : 0.f;
            rs[k] = ok ? rstd[row] : 0.f;
            const float* xr = x + (long)row * ldx;
            const float* dyr = dy + (long)row * lddy;
#pragma unroll
            for (int c = 0; c < VPL; ++c) {
                const int col = (lane + 64 * c) * 4;
                const bool in = ok && col < D;
                xv[k][c] = in ? *reinterpret_cast<const float4*>(xr + col) : make_float4(0.f, 0.f, 0.f, 0.f);
                d[k][c] = in ? *reinterpret_cast<const float4*>(dyr + col) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int k = 0; k < RPI; ++k) {
            const int row = r0 + k * S;
            if (row >= rows) break;
            float4 xh[VPL], g[VPL];
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int c = 0; c < VPL; ++c) {
                const int col = (lane + 64 * c) * 4;
                if (col < D) {
                    const float m = mu[k], q = rs[k];
                    xh[c] = make_float4((xv[k][c].x - m) * q, (xv[k][c].y - m) * q, (xv[k][c].z - m) * q,
                                        (xv[k][c].w - m) * q);
                    const float4 dd = d[k][c];
                    g[c] = make_float4(dd.x * wv[c].x, dd.y * wv[c].y, dd.z * wv[c].z, dd.w * wv[c].w);
                    s1 += (g[c].x + g[c].y) + (g[c].z + g[c].w);
                    s2 += (g[c].x * xh[c].x + g[c].y * xh[c].y) + (g[c].z * xh[c].z + g[c].w * xh[c].w);
                    aw[c].x += dd.x * xh[c].x; aw[c].y += dd.y * xh[c].y;
                    aw[c].z += dd.z * xh[c].z; aw[c].w += dd.w * xh[c].w;
                    ab[c].x += dd.x; ab[c].y += dd.y; ab[c].z += dd.z; ab[c].w += dd.w;
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
                    o.x = (g[c].x - m1 - xh[c].x * m2) * rs[k];
                    o.y = (g[c].y - m1 - xh[c].y * m2) * rs[k];
                    o.z = (g[c].z - m1 - xh[c].z * m2) * rs[k];
                    o.w = (g[c].w - m1 - xh[c].w * m2) * rs[k];
                    if (dr) {
                        const float4 rv = *reinterpret_cast<const float4*>(dr + col);
                        o.x += rv.x; o.y += rv.y; o.z += rv.z; o.w += rv.w;
                    }
                    *reinterpret_cast<float4*>(dxr + col) = o;
                    if (dxh) st_bf16x4(dxh, (long)row * lddx + col, o);
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
        sh_w[wave][lane + 64 * c] = aw[c];
        sh_b[wave][lane + 64 * c] = ab[c];
    }
    __syncthreads();
    // wave 0 folds the waves in fixed order and writes this block's partial
    if (wave == 0) {
        float* pw = part + (long)blockIdx.x * 2 * D;
#pragma unroll
        for (int c = 0; c < VPL; ++c) {
            const int col = (lane + 64 * c) * 4;
            if (col < D) {
                float4 sw = sh_w[0][lane + 64 * c], sb = sh_b[0][lane + 64 * c];
                for (int k = 1; k < WPB; ++k) {
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
              float* mean, float* rstd, int rows, int D, hipStream_t s, const int* rows_dev, int ybf) {
    PT_REQUIRE(D >= 1 && D <= 1024, "layernorm: D=%d unsupported", D);
    const bool vec = ln_vec_ok(x, ldx, D) && ln_vec_ok(y, ldy, D) && ln_vec_ok(w, 0, D) && ln_vec_ok(b, 0, D);
    if (ybf) {
        PT_REQUIRE(vec && D <= 256, "layernorm: bf16 output needs D <= 256, multiples of 4, 16 B aligned rows");
        const int slot = pt_prof_open(s);
        hipLaunchKernelGGL((ln_fwd_kernel<1, LN_FWD_RPW, true>), dim3(pt_cdiv(rows, 4 * LN_FWD_RPW)), dim3(256), 0,
                           s, x, ldx, w, b, y, ldy, mean, rstd, rows, D, rows_dev);
        PT_LAUNCH_CHECK();
        pt_prof_close(slot, PROF_LN_FWD, (double)rows * (6.0 * D + 8.0) + 8.0 * D, s);
        return PTCG_OK;
    }
    const int slot = pt_prof_open(s);
    if (!vec) {
        hipLaunchKernelGGL(ln_fwd_scalar_kernel, dim3(pt_cdiv(rows, 4)), dim3(256), 0, s, x, ldx, w, b, y, ldy,
                           mean, rstd, rows, D, rows_dev);
    } else {
        const dim3 grid(pt_cdiv(rows, 4 * LN_FWD_RPW));
        if (D <= 256)
            hipLaunchKernelGGL((ln_fwd_kernel<1, LN_FWD_RPW>), grid, dim3(256), 0, s, x, ldx, w, b, y, ldy, mean,
                               rstd, rows, D, rows_dev);
        else if (D <= 512)
            hipLaunchKernelGGL((ln_fwd_kernel<2, LN_FWD_RPW>), grid, dim3(256), 0, s, x, ldx, w, b, y, ldy, mean,
                               rstd, rows, D, rows_dev);
        else
            hipLaunchKernelGGL((ln_fwd_kernel<4, LN_FWD_RPW>), grid, dim3(256), 0, s, x, ldx, w, b, y, ldy, mean,
                               rstd, rows, D, rows_dev);
    }
    PT_LAUNCH_CHECK();
    // read x, write y, mean, rstd; read w, b
    pt_prof_close(slot, PROF_LN_FWD, (double)rows * (8.0 * D + 8.0) + 8.0 * D, s);
    return PTCG_OK;
}

int pt_ln_bwd(const float* dy, long lddy, const float* x, long ldx, const float* w,
              const float* mean, const float* rstd, const float* dres, long ldres, float* dx,
              long lddx, float* dw, float* db, int rows, int D, float* ws, long ws_floats,
              hipStream_t s, const int* rows_dev, float* dxh) {
    PT_REQUIRE(D >= 1 && D <= 1024, "layernorm bwd: D=%d unsupported", D);
    const bool vec = ln_vec_ok(dy, lddy, D) && ln_vec_ok(x, ldx, D) && ln_vec_ok(w, 0, D) &&
                     ln_vec_ok(dx, lddx, D) && (dres == nullptr || ln_vec_ok(dres, ldres, D));
    PT_REQUIRE(!dxh || (vec && ((uintptr_t)dxh & 15) == 0), "layernorm bwd: bf16 copy needs the vector layout");
    // 8-wave workgroups for the d <= 256 rows (16 KB of fold buffers);
    // 4-wave ones for wider rows and the scalar kernel
    const int wpb = (vec && D <= 256) ? LN_BWD_WPB : 4;
    int blocks = pt_cdiv(rows, wpb);
    if (blocks > LN_BWD_BLOCKS) blocks = LN_BWD_BLOCKS;
    if (blocks < 1) blocks = 1;
    PT_REQUIRE(ws && (long)blocks * 2 * D * 2 <= ws_floats, "layernorm bwd: workspace too small");
    const dim3 grid(blocks), blk(64 * wpb);
    const int slot = pt_prof_open(s);
    if (!vec)
        hipLaunchKernelGGL(ln_bwd_scalar_kernel, grid, blk, 0, s, dy, lddy, x, ldx, w, mean, rstd, dres, ldres, dx,
                           lddx, ws, rows, D, rows_dev);
    else if (D <= 256)
        hipLaunchKernelGGL((ln_bwd_kernel<1, LN_BWD_WPB, LN_BWD_RPI>), grid, blk, 0, s, dy, lddy, x, ldx, w, mean,
                           rstd, dres, ldres, dx, lddx, ws, rows, D, rows_dev, dxh);
    else if (D <= 512)
        hipLaunchKernelGGL((ln_bwd_kernel<2, 4, LN_BWD_RPI>), grid, blk, 0, s, dy, lddy, x, ldx, w, mean, rstd, dres,
                           ldres, dx, lddx, ws, rows, D, rows_dev, dxh);
    else
        hipLaunchKernelGGL((ln_bwd_kernel<4, 4, LN_BWD_RPI>), grid, blk, 0, s, dy, lddy, x, ldx, w, mean, rstd, dres,
                           ldres, dx, lddx, ws, rows, D, rows_dev, dxh);
    PT_LAUNCH_CHECK();
    // read dy, x, mean, rstd (and dres), write dx (and its bf16 copy); read w, write dW, dB
    pt_prof_close(slot, PROF_LN_BWD,
                  (double)rows * (12.0 * D + 8.0 + (dres ? 4.0 * D : 0.0) + (dxh ? 2.0 * D : 0.0)) + 12.0 * D, s);
    if (dw && db)
        return pt_colsum2(ws, 2 * D, blocks, 2 * D, D, dw, db, ws + (long)blocks * 2 * D,
                          ws_floats - (long)blocks * 2 * D, s);
    PT_REQUIRE(!dw && !db, "layernorm bwd: dw and db must both be given or both be NULL");
    return PTCG_OK;
}
