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
