// Rollout-side steps around the training step: the train-layout transpose,
// the negamax V-trace/GAE advantage, prioritized segment replay and the
// index copy of per-minibatch results back into the rollout.
//
// Replaces, from train_impl (native/src/pufferlib.cu:1847-2160):
//   transpose_102 + clamp_precision_kernel + fill_precision_kernel
//     (:1863-1895; native/src/kernels.cu:179-203)   -> ptcg_transpose_102, ptcg_fill
//   puf_zero + ptcg_puff_advantage / k_negamax_adv
//     (:1966-1973; native/model/ptcg_model2.cu:287-321) -> ptcg_negamax_advantage
//   prio_replay_cuda (:1455-1591)                   -> ptcg_prio_replay
//   select_copy (:1777-1826)                        -> row indices: the step reads
//                                                      its rows through row_idx
//   index_copy (:1747-1754, :2146-2160)             -> ptcg_index_copy
//
// Layout choices:
// * transpose: rows of C floats move whole (one wave per row, 128-bit) when
//   C % 4 == 0; C == 1 goes through a 64 x 64 LDS tile so both sides are
//   coalesced; the reward clamp is fused into the rewards' transpose.
// * advantage: one wave per segment, lane = time step, so the loads of a
//   segment's 64 steps (and the 64 strided seat reads from obs) are issued
//   together; the backward recurrence then runs over the lanes in order
//   (v_readlane), with the reference's arithmetic in the reference's order.
//   The reference runs one thread per segment over 64 dependent iterations.
// * replay: |adv| row sums one wave per segment, then ONE workgroup
//   normalizes, scans (block-wide, in LDS), draws and weights (the reference
//   uses 6 launches including a single-thread serial CDF).
#include "model.h"

namespace {

__device__ __forceinline__ float clamp_unit(float v) { return fminf(fmaxf(v, -1.f), 1.f); }

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// [A, B, C] -> [B, A, C] for C % 4 == 0: one wave per source row (a, b)
__global__ __launch_bounds__(256) void transpose_rows_kernel(float4* __restrict__ dst, const float4* __restrict__ src,
                                                             int A, int B, int C4, int clamp) {
    const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= (long)A * B) return;
    const long a = row / B, b = row % B;
    const float4* s = src + row * C4;
    float4* d = dst + (b * A + a) * C4;
    for (int i = threadIdx.x & 63; i < C4; i += 64) {
        float4 v = s[i];
        if (clamp) {
            v.x = clamp_unit(v.x);
            v.y = clamp_unit(v.y);
            v.z = clamp_unit(v.z);
            v.w = clamp_unit(v.w);
        }
        d[i] = v;
    }
}

// [A, B] -> [B, A] through a 64 x 65 LDS tile
__global__ __launch_bounds__(256) void transpose_2d_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                           int A, int B, int clamp) {
    __shared__ float tile[64][65];
    const int a0 = blockIdx.y * 64, b0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4) {
        const int a = a0 + r, b = b0 + tx;
        if (a < A && b < B) {
            const float v = src[(long)a * B + b];
            tile[r][tx] = clamp ? clamp_unit(v) : v;
        }
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        const int b = b0 + r, a = a0 + tx;
        if (a < A && b < B) dst[(long)b * A + a] = tile[tx][r];
    }
}

// any C: element-wise, grid-stride
__global__ __launch_bounds__(256) void transpose_elem_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                             int A, int B, int C, int clamp) {
    const long n = (long)A * B * C, BC = (long)B * C;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const long a = i / BC, rem = i % BC, b = rem / C, c = rem % C;
        const float v = src[i];
        dst[(b * A + a) * C + c] = clamp ? clamp_unit(v) : v;
    }
}

__global__ __launch_bounds__(256) void fill_kernel(float* __restrict__ p, long n, float v) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) p[i] = v;
}

// Negamax V-trace/GAE over rows of T steps ((B, T) layout, row-major):
//   s_t     = (seat_t == seat_{t+1} ? 1 : -1) * (1 - done_{t+1})
//   delta_t = min(imp_t, rho_clip) * (r_{t+1} + gamma v_{t+1} s_t - v_t)
//   A_t     = delta_t + gamma lambda min(imp_t, c_clip) s_t A_{t+1},  A_{T-1} = 0
// seat_t = obs[(row * T + t) * obs_stride + seat_col].  One wave per row;
// steps in chunks of 64 from the end, step t+1 of a chunk's last lane
// carried from the chunk after it.
constexpr int ADV_WAVES = 4;

__global__ __launch_bounds__(64 * ADV_WAVES) void negamax_adv_kernel(
        const float* __restrict__ values, const float* __restrict__ rewards, const float* __restrict__ dones,
        const float* __restrict__ importance, const float* __restrict__ obs, long obs_stride, int seat_col,
        float* __restrict__ adv, float* __restrict__ returns, float gamma, float lambda, float rho_clip,
        float c_clip, int B, int T) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * ADV_WAVES + (threadIdx.x >> 6);
    if (row >= B) return;
    const long o = (long)row * T;
    float lastlam = 0.f;
    float c_seat = 0.f, c_v = 0.f, c_r = 0.f, c_d = 0.f;   // step 64(c+1) of the chunk after
    for (int c = (T - 1) / 64; c >= 0; --c) {
        const int t = c * 64 + lane;
        float seat = 0.f, v = 0.f, r = 0.f, d = 0.f, imp = 0.f;
        if (t < T) {
            seat = obs[(o + t) * obs_stride + seat_col];
            v = values[o + t];
            r = rewards[o + t];
            d = dones[o + t];
            imp = importance[o + t];
        }
        float seat_n = __shfl_down(seat, 1, 64), v_n = __shfl_down(v, 1, 64);
        float r_n = __shfl_down(r, 1, 64), d_n = __shfl_down(d, 1, 64);
        if (lane == 63) {
            seat_n = c_seat;
            v_n = c_v;
            r_n = c_r;
            d_n = c_d;
        }
        c_seat = readlane_f(seat, 0);
        c_v = readlane_f(v, 0);
        c_r = readlane_f(r, 0);
        c_d = readlane_f(d, 0);
        const float sign = seat == seat_n ? 1.f : -1.f;
        const float s = sign * (1.f - d_n);
        const float rho = imp < rho_clip ? imp : rho_clip;
        const float cc = imp < c_clip ? imp : c_clip;
        const float delta = rho * (r_n + gamma * v_n * s - v);
        const float coef = gamma * lambda * cc * s;
        const int last = min(63, T - 2 - c * 64);   // last lane of the chunk with t <= T-2
        float mine = 0.f;
        for (int j = last; j >= 0; --j) {
            lastlam = readlane_f(delta, j) + readlane_f(coef, j) * lastlam;
            if (lane == j) mine = lastlam;
        }
        if (t < T) {
            adv[o + t] = mine;
            if (returns) returns[o + t] = v + mine;
        }
    }
}

// prioritized replay, pass 1: p_b = (sum_t |adv_bt|)^alpha, non-finite -> 0
__global__ __launch_bounds__(256) void prio_rowsum_kernel(const float* __restrict__ adv, float* __restrict__ pw,
                                                          int B, int T, float alpha) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= B) return;
    const float* a = adv + (long)row * T;
    float s = 0.f;
    for (int t = threadIdx.x & 63; t < T; t += 64) s += fabsf(a[t]);
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) {
        float p = powf(s, alpha);
        if (isnan(p) || isinf(p)) p = 0.f;
        pw[row] = p;
    }
}

constexpr int PRIO_NT = 1024;
constexpr float PRIO_EPS = 1e-6f;

// pass 2, one workgroup: probs = (p + eps) / (sum p + eps); cdf = inclusive
// scan; n draws u_k = Philox(counter = (offset + k, 0, 1), key = seed) ->
// idx_k = first b with cdf_b >= u_k (B-1 if none); weight_k =
// (total_agents * probs[idx_k])^-beta; offset += n.  Dynamic LDS: 2 B floats.
__global__ __launch_bounds__(PRIO_NT) void prio_sample_kernel(
        float* __restrict__ probs, float* __restrict__ cdf, int B, int T, int n_samples, int total_agents,
        float beta, unsigned long long seed, long long* __restrict__ offset, int32_t* __restrict__ idx,
        float* __restrict__ mb_prio, int32_t* __restrict__ row_idx, float* __restrict__ row_prio) {
    extern __shared__ float sh[];
    float* sp = sh;        // normalized probabilities
    float* sc = sh + B;    // CDF
    __shared__ float wsum[PRIO_NT / 64];
    __shared__ float s_total;
    __shared__ long long s_off;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float s = 0.f;
    for (int i = tid; i < B; i += PRIO_NT) s += probs[i];
    s = wave_sum(s);
    if (lane == 0) wsum[wave] = s;
    __syncthreads();
    if (tid == 0) {
        float t = 0.f;
        for (int w = 0; w < PRIO_NT / 64; ++w) t += wsum[w];
        s_total = t + PRIO_EPS;
        s_off = *offset;
    }
    __syncthreads();
    const float total = s_total;
    for (int i = tid; i < B; i += PRIO_NT) {
        const float p = (probs[i] + PRIO_EPS) / total;
        sp[i] = p;
        probs[i] = p;
    }
    __syncthreads();
    // block-wide inclusive scan: thread tid owns a contiguous chunk
    const int per = (B + PRIO_NT - 1) / PRIO_NT;
    const int i0 = min(B, tid * per), i1 = min(B, i0 + per);
    float run = 0.f;
    for (int i = i0; i < i1; ++i) run += sp[i];
    float incl = run;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    float excl = __shfl_up(incl, 1, 64);
    if (lane == 0) excl = 0.f;
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    float acc = 0.f;
    for (int w = 0; w < wave; ++w) acc += wsum[w];
    acc += excl;
    for (int i = i0; i < i1; ++i) {
        acc += sp[i];
        sc[i] = acc;
        cdf[i] = acc;
    }
    __syncthreads();
    for (int k = tid; k < n_samples; k += PRIO_NT) {
        const unsigned long long draw = (unsigned long long)s_off + (unsigned long long)k;
        const uint4 r = philox4x32_10(make_uint4((unsigned)draw, (unsigned)(draw >> 32), 0u, 1u),
                                      make_uint2((unsigned)seed, (unsigned)(seed >> 32)));
        const float u = pt_u01(r.x);
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (sc[mid] < u) lo = mid + 1;
            else hi = mid;
        }
        const float w = powf(sp[lo] * (float)total_agents, -beta);
        idx[k] = lo;
        if (mb_prio) mb_prio[k] = w;
        for (int t = 0; t < T; ++t) {
            if (row_idx) row_idx[(long)k * T + t] = lo * T + t;
            if (row_prio) row_prio[(long)lo * T + t] = w;
        }
    }
    if (tid == 0) *offset = s_off + n_samples;
}

// dst row idx[i] (row_floats floats) <- src row i; rows with idx outside
// [0, dst_rows) are skipped.  One wave per row.
__global__ __launch_bounds__(256) void index_copy_kernel(float* __restrict__ dst, const int32_t* __restrict__ idx,
                                                         const float* __restrict__ src, int n_idx, int row_floats,
                                                         int dst_rows) {
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= n_idx) return;
    const int r = idx[i];
    if (r < 0 || r >= dst_rows) return;
    float* d = dst + (long)r * row_floats;
    const float* s = src + (long)i * row_floats;
    for (int c = threadIdx.x & 63; c < row_floats; c += 64) d[c] = s[c];
}

// segments whose probabilities and CDF fit one workgroup's LDS (64 KB less
// the static arrays)
constexpr int PRIO_MAX_SEGMENTS = (65536 - 1024) / 8;

}  // namespace

extern "C" int ptcg_transpose_102(float* dst, const float* src, int A, int B, int C, int clamp, void* stream) {
    PT_REQUIRE(dst && src, "transpose_102: null buffer");
    PT_REQUIRE(A >= 1 && B >= 1 && C >= 1, "transpose_102: bad shape (%d, %d, %d)", A, B, C);
    PT_REQUIRE(dst != src, "transpose_102: dst and src must not alias");
    hipStream_t s = (hipStream_t)stream;
    const long rows = (long)A * B;
    if (C % 4 == 0 && (((uintptr_t)dst | (uintptr_t)src) & 15) == 0) {
        PT_REQUIRE((rows + 3) / 4 <= 0x7fffffffL, "transpose_102: too many rows");
        hipLaunchKernelGGL(transpose_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, (float4*)dst,
                           (const float4*)src, A, B, C / 4, clamp);
    } else if (C == 1) {
        PT_REQUIRE(pt_cdiv(A, 64) <= 65535, "transpose_102: A=%d too large", A);
        hipLaunchKernelGGL(transpose_2d_kernel, dim3(pt_cdiv(B, 64), pt_cdiv(A, 64)), dim3(256), 0, s, dst, src, A,
                           B, clamp);
    } else {
        const long n = rows * C;
        long blocks = (n + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(transpose_elem_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, src, A, B, C, clamp);
    }
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

extern "C" int ptcg_fill(float* dst, int64_t n, float value, void* stream) {
    PT_REQUIRE(dst && n >= 0, "fill: bad arguments");
    if (n == 0) return PTCG_OK;
    long blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, dst, (long)n, value);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

extern "C" int ptcg_negamax_advantage(const float* values, const float* rewards, const float* dones,
                                      const float* importance, const float* obs, int64_t obs_stride, int seat_col,
                                      float* advantages, float* returns, float gamma, float lambda, float rho_clip,
                                      float c_clip, int B, int T, void* stream) {
    PT_REQUIRE(values && rewards && dones && importance && obs && advantages, "negamax_advantage: null buffer");
    PT_REQUIRE(B >= 1 && T >= 1, "negamax_advantage: bad shape (%d, %d)", B, T);
    PT_REQUIRE(seat_col >= 0 && seat_col < obs_stride, "negamax_advantage: seat column %d outside rows of %ld",
               seat_col, (long)obs_stride);
    hipLaunchKernelGGL(negamax_adv_kernel, dim3(pt_cdiv(B, ADV_WAVES)), dim3(64 * ADV_WAVES), 0,
                       (hipStream_t)stream, values, rewards, dones, importance, obs, (long)obs_stride, seat_col,
                       advantages, returns, gamma, lambda, rho_clip, c_clip, B, T);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

extern "C" int ptcg_prio_replay_max_segments(void) { return PRIO_MAX_SEGMENTS; }

extern "C" int ptcg_prio_replay(const float* advantages, int B, int T, float prio_alpha, int n_samples,
                                int total_agents, float anneal_beta, uint64_t seed, int64_t* rng_offset,
                                float* probs, float* cdf, int32_t* idx, float* mb_prio, int32_t* row_idx,
                                float* row_prio, void* stream) {
    PT_REQUIRE(advantages && probs && cdf && idx && rng_offset, "prio_replay: null buffer");
    PT_REQUIRE(B >= 1 && T >= 1 && n_samples >= 1, "prio_replay: bad sizes (B %d, T %d, samples %d)", B, T,
               n_samples);
    PT_REQUIRE(B <= PRIO_MAX_SEGMENTS, "prio_replay: %d segments exceed one workgroup's LDS (at most %d)", B,
               PRIO_MAX_SEGMENTS);
    PT_REQUIRE((long)B * T <= 0x7fffffffL, "prio_replay: B*T too large");
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(prio_rowsum_kernel, dim3(pt_cdiv(B, 4)), dim3(256), 0, s, advantages, probs, B, T, prio_alpha);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(prio_sample_kernel, dim3(1), dim3(PRIO_NT), (size_t)B * 8, s, probs, cdf, B, T, n_samples,
                       total_agents, anneal_beta, (unsigned long long)seed, (long long*)rng_offset, idx, mb_prio,
                       row_idx, row_prio);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

extern "C" int ptcg_index_copy(float* dst, const int32_t* idx, const float* src, int n_idx, int row_floats,
                               int dst_rows, void* stream) {
    PT_REQUIRE(dst && idx && src, "index_copy: null buffer");
    PT_REQUIRE(n_idx >= 0 && row_floats >= 1 && dst_rows >= 1, "index_copy: bad sizes");
    if (n_idx == 0) return PTCG_OK;
    hipLaunchKernelGGL(index_copy_kernel, dim3(pt_cdiv(n_idx, 4)), dim3(256), 0, (hipStream_t)stream, dst, idx, src,
                       n_idx, row_floats, dst_rows);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
