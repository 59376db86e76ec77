// Action sampler for rollouts: one counter-based uniform per row, inverse
// CDF over the masked softmax of the option scores.
//
// Replaces sample_logits (native/src/pufferlib.cu:584-718) for one discrete
// head: logits made safe (NaN -> 0, +-inf -> +-3.4028e38), options with
// mask == 0 -> -1e4 (masked_logit :548-557), online max / sum-exp, walk of
// exp(l - logsumexp) until the running sum exceeds u, fallback to the last
// legal option; logprob = l[a] - logsumexp; value = the fused last column.
// The reference draws u from a per-row cuRAND state it stores and advances;
// here u comes from Philox4x32-10 (Salmon et al., SC'11, restated from the
// paper) keyed by (seed, step, row), so a rollout step needs no RNG state in
// memory and any (step, row) can be replayed.
#include "model.h"

namespace {

__device__ __forceinline__ float safe_masked(float l, const float* mk, int a) {
    if (isnan(l)) l = 0.f;
    if (isinf(l)) l = l > 0.f ? 3.4028e+38f : -3.4028e+38f;
    if (mk && mk[a] == 0.f) l = -1e4f;
    return l;
}

__global__ void sample_kernel(const float* __restrict__ dec, int n, int A, const float* __restrict__ mask,
                              long mstride, const int32_t* __restrict__ idx, unsigned long long seed,
                              unsigned long long step, const unsigned long long* __restrict__ step_dev,
                              float* __restrict__ actions, float* __restrict__ logprobs,
                              float* __restrict__ values, float* __restrict__ uniforms) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (step_dev) step = *step_dev;   // a captured rollout reads its step at replay time
    const float* l = dec + (long)i * (A + 1);
    const float* mk = mask ? mask + (idx ? (long)idx[i] : (long)i) * mstride : nullptr;
    float mx = -INFINITY, se = 0.f;
    for (int a = 0; a < A; ++a) {
        const float v = safe_masked(l[a], mk, a);
        if (v > mx) {
            se *= expf(mx - v);
            mx = v;
        }
        se += expf(v - mx);
    }
    const float lse = mx + logf(se);
    const uint4 r = philox4x32_10(make_uint4((unsigned)i, (unsigned)step, (unsigned)(step >> 32), 0u),
                                  make_uint2((unsigned)seed, (unsigned)(seed >> 32)));
    const float u = pt_u01(r.x);
    float cs = 0.f;
    int act = -1;
    for (int a = 0; a < A; ++a) {
        cs += expf(safe_masked(l[a], mk, a) - lse);
        if (u < cs) {
            act = a;
            break;
        }
    }
    if (act < 0) {
        act = A - 1;
        if (mk)
            for (int a = A - 1; a >= 0; --a)
                if (mk[a] != 0.f) {
                    act = a;
                    break;
                }
    }
    actions[i] = (float)act;
    logprobs[i] = safe_masked(l[act], mk, act) - lse;
    if (values) values[i] = l[A];
    if (uniforms) uniforms[i] = u;
}

// advances a captured rollout's step counter after its draws
__global__ void step_advance_kernel(unsigned long long* step_dev) { step_dev[0] += 1ull; }

// ---- Gumbel-max sampling (no counterpart in the reference, whose rollout
// draws by inverse CDF): a = argmax_j (l_j + g_j) over the safe, masked
// logits, g_j = -log(-log u_j), u_j = Philox4x32-10 with counter
// (row, step lo, step hi, 1 + j/4), word j % 4, key = seed.  The logarithm is
// pt_log_rep: only correctly rounded fp32 +, -, *, / in a fixed order (no
// fused multiply-add), so a CPU restatement in IEEE fp32 reproduces every
// noise value and every draw bit for bit.
//
// pt_log_rep(x), x > 0 normal: x = m 2^e with m in [sqrt(1/2), sqrt(2)),
// log m = 2 atanh(s) = 2 s (1 + z/3 + z^2/5 + ... + z^5/11), s = (m-1)/(m+1),
// z = s^2 (|s| <= 0.1716, truncation < 1e-9 relative), log x = e ln2_hi +
// (log m + e ln2_lo) with ln2 split so that e ln2_hi is exact.  The classic
// argument reduction + atanh series (Abramowitz & Stegun 4.1.27).
__device__ float pt_log_rep(float x) {
#pragma clang fp contract(off)
    const unsigned b = __float_as_uint(x);
    int e = (int)(b >> 23) - 127;
    unsigned mb = (b & 0x007fffffu) | 0x3f800000u;
    if (mb > 0x3fb504f3u) {   // m > sqrt(2): halve it (exact)
        mb -= 0x00800000u;
        e += 1;
    }
    const float m = __uint_as_float(mb);
    const float s = (m - 1.0f) / (m + 1.0f);
    const float z = s * s;
    float p = 0.0909090936f;                 // 1/11
    p = 0.111111112f + z * p;                // 1/9
    p = 0.142857149f + z * p;                // 1/7
    p = 0.200000003f + z * p;                // 1/5
    p = 0.333333343f + z * p;                // 1/3
    p = 1.0f + z * p;
    const float lm = (s + s) * p;
    const float ef = (float)e;
    return ef * 0.693145752f + (lm + ef * 1.42860677e-06f);
}

__device__ __forceinline__ float pt_gumbel(float u) { return -pt_log_rep(-pt_log_rep(u)); }

// one wave per row (lane = option, A <= 64), four rows per workgroup
__global__ __launch_bounds__(256) void gumbel_sample_kernel(const float* __restrict__ dec, int n, int A,
        const float* __restrict__ mask, long mstride, const int32_t* __restrict__ idx,
        const float* __restrict__ noise, unsigned long long seed, unsigned long long step,
        const unsigned long long* __restrict__ step_dev, float* __restrict__ actions,
        float* __restrict__ logprobs, float* __restrict__ values, float* __restrict__ noise_out) {
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= n) return;
    if (step_dev) step = *step_dev;
    const float* l = dec + (long)i * (A + 1);
    const float* mk = mask ? mask + (idx ? (long)idx[i] : (long)i) * mstride : nullptr;
    const bool on = lane < A;
    const float v = on ? safe_masked(l[lane], mk, lane) : -INFINITY;
    float g = 0.f;
    if (on) {
        if (noise) {
            g = noise[(long)i * A + lane];
        } else {
            const uint4 r = philox4x32_10(make_uint4((unsigned)i, (unsigned)step, (unsigned)(step >> 32),
                                                     1u + (unsigned)(lane >> 2)),
                                          make_uint2((unsigned)seed, (unsigned)(seed >> 32)));
            const unsigned w = (lane & 3) == 0 ? r.x : (lane & 3) == 1 ? r.y : (lane & 3) == 2 ? r.z : r.w;
            g = pt_gumbel(pt_u01(w));
        }
        if (noise_out) noise_out[(long)i * A + lane] = g;
    }
    // argmax of v + g; ties go to the lowest option index
    float best = on ? v + g : -INFINITY;
    int arg = on ? lane : 0x7fffffff;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o, 64);
        const int oa = __shfl_xor(arg, o, 64);
        if (ob > best || (ob == best && oa < arg)) {
            best = ob;
            arg = oa;
        }
    }
    // log-probability of the draw under the masked softmax
    const float mx = wave_max(v);
    const float se = wave_sum(on ? expf(v - mx) : 0.f);
    const float lse = mx + logf(se);
    const float va = __shfl(v, arg, 64);
    if (lane == 0) {
        actions[i] = (float)arg;
        logprobs[i] = va - lse;
        if (values) values[i] = l[A];
    }
}

}  // namespace

int pt_sample_actions_dev(const float* dec_out, int n, int A, const float* mask, long mask_stride,
                          const int32_t* row_idx, uint64_t seed, uint64_t* step_dev, float* actions,
                          float* logprobs, float* values, hipStream_t s) {
    PT_REQUIRE(dec_out && actions && logprobs && step_dev, "sample_actions: null buffer");
    PT_REQUIRE(n > 0 && A > 0, "sample_actions: empty shape n=%d A=%d", n, A);
    hipLaunchKernelGGL(sample_kernel, dim3(pt_cdiv(n, 256)), dim3(256), 0, s, dec_out, n, A, mask, mask_stride,
                       row_idx, (unsigned long long)seed, 0ull, (const unsigned long long*)step_dev, actions,
                       logprobs, values, (float*)nullptr);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(step_advance_kernel, dim3(1), dim3(1), 0, s, (unsigned long long*)step_dev);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}

int pt_sample_gumbel(const float* dec_out, int n, int A, const float* mask, long mask_stride,
                     const int32_t* row_idx, const float* noise, uint64_t seed, uint64_t step,
                     uint64_t* step_dev, float* actions, float* logprobs, float* values, float* noise_out,
                     hipStream_t s) {
    PT_REQUIRE(dec_out && actions && logprobs, "sample_gumbel: null buffer");
    PT_REQUIRE(n > 0 && A > 0 && A <= 64, "sample_gumbel: shape n=%d A=%d (1 <= A <= 64)", n, A);
    hipLaunchKernelGGL(gumbel_sample_kernel, dim3(pt_cdiv(n, 4)), dim3(256), 0, s, dec_out, n, A, mask, mask_stride,
                       row_idx, noise, (unsigned long long)seed, (unsigned long long)step,
                       (const unsigned long long*)step_dev, actions, logprobs, values, noise_out);
    PT_LAUNCH_CHECK();
    if (step_dev) {
        hipLaunchKernelGGL(step_advance_kernel, dim3(1), dim3(1), 0, s, (unsigned long long*)step_dev);
        PT_LAUNCH_CHECK();
    }
    return PTCG_OK;
}

extern "C" int ptcg_sample_actions_gumbel(const float* dec_out, int n, int A, const float* mask,
                                          int64_t mask_stride, const int32_t* row_idx, const float* noise,
                                          uint64_t seed, uint64_t step, float* actions, float* logprobs,
                                          float* values, float* noise_out, void* stream) {
    return pt_sample_gumbel(dec_out, n, A, mask, (long)mask_stride, row_idx, noise, seed, step, nullptr, actions,
                            logprobs, values, noise_out, (hipStream_t)stream);
}

extern "C" int ptcg_sample_actions(const float* dec_out, int n, int A, const float* mask, int64_t mask_stride,
                                   const int32_t* row_idx, uint64_t seed, uint64_t step, float* actions,
                                   float* logprobs, float* values, float* uniforms, void* stream) {
    PT_REQUIRE(dec_out && actions && logprobs, "sample_actions: null buffer");
    PT_REQUIRE(n > 0 && A > 0, "sample_actions: empty shape n=%d A=%d", n, A);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(sample_kernel, dim3(pt_cdiv(n, 256)), dim3(256), 0, s, dec_out, n, A, mask, (long)mask_stride,
                       row_idx, (unsigned long long)seed, (unsigned long long)step,
                       (const unsigned long long*)nullptr, actions, logprobs, values, uniforms);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
