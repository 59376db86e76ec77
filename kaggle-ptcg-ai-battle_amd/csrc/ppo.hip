// PPO clipped-surrogate + clipped value + entropy loss, forward statistics
// and hand-written gradient, for one discrete head of A <= 64 options.
//
// Same formulas as the reference's ppo_var_mean / ppo_discrete_head /
// ppo_loss_compute / ppo_loss_reduce (native/src/pufferlib.cu:949-1363),
// T_seq = 1 and no league tag: advantage normalised per minibatch with the
// unbiased variance, mask == 0 -> logit -1e4, ratio = exp(logp - old_logp),
// pg = max(-w adv_n r, -w adv_n clip(r)), v_loss = 0.5 max((v-R)^2,
// (v_old + clip(v - v_old) - R)^2), everything / N.  Layout differs: a
// wave64 takes four rows with lane = option (the reference runs one thread
// per row over a serial 64-option loop), and the advantage statistics are
// computed redundantly by every workgroup in the same fixed order, while its
// rows' loads are in flight, instead of by a separate <<<1,256>>> kernel, so
// the step is two launches.
#include "common.h"

namespace {

constexpr int NSTAT = 7;   // pg, vf, ent, total, old_approx_kl, approx_kl, clipfrac

struct PPOArgs {
    const float* out; int n, A;
    const float* mask; long mask_stride;
    const int32_t* idx;
    const float *actions, *old_logp, *adv, *ret, *val, *prio;
    float clip, vf_clip, vf_coef;
    const float* ent_coef;   // device scalar (the reference's *a.ent_coef, pufferlib.cu:1063)
    float *grad, *ratio, *newvalue, *partial;
};

__device__ __forceinline__ int rix(const int32_t* idx, int r) { return idx ? idx[r] : r; }

// rows per wave and per workgroup (four waves)
constexpr int RPW = 4, RPB = 4 * RPW;

// block-wide sum of one value per thread: wave sums, then the four waves in
// order (every workgroup gets the same bits)
__device__ __forceinline__ float block_sum4(float v, float* red, int tid) {
    v = wave_sum(v);
    __syncthreads();   // red is free (a previous call's readers are done)
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

__global__ __launch_bounds__(256) void ppo_loss_kernel(PPOArgs a) {
    __shared__ float red[4];
    __shared__ float rowstat[4][NSTAT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int A = a.A;
    const bool on = lane < A;
    // this wave's rows: logits, mask and per-row inputs are loaded first, so
    // they are in flight while the advantage statistics are formed
    const int r0 = blockIdx.x * RPB + wave * RPW;
    float l[RPW], vpred[RPW], old_logp[RPW], adv[RPW], w[RPW], vold[RPW], ret[RPW];
    int act[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const int r = r0 + j < a.n ? r0 + j : a.n - 1;   // clamped: rows past n are loaded, not used
        const int src = rix(a.idx, r);
        const float* lg = a.out + (long)r * (A + 1);
        const float* mk = a.mask + (long)src * a.mask_stride;
        l[j] = -INFINITY;
        if (on) l[j] = (mk[lane] == 0.f) ? -1e4f : lg[lane];
        vpred[j] = lg[A];
        act[j] = (int)a.actions[src];
        old_logp[j] = a.old_logp[src];
        adv[j] = a.adv[src];
        w[j] = a.prio ? a.prio[src] : 1.0f;
        vold[j] = a.val[src];
        ret[j] = a.ret[src];
    }
    // minibatch advantage mean / unbiased variance (pufferlib.cu:1307-1363),
    // two passes over the rows, computed alike by every workgroup
    float s0 = 0.f, s1 = 0.f;
    int i = tid;
    for (; i + 256 < a.n; i += 512) {
        s0 += a.adv[rix(a.idx, i)];
        s1 += a.adv[rix(a.idx, i + 256)];
    }
    if (i < a.n) s0 += a.adv[rix(a.idx, i)];
    const float mean = block_sum4(s0 + s1, red, tid) / (float)a.n;
    float q0 = 0.f, q1 = 0.f;
    for (i = tid; i + 256 < a.n; i += 512) {
        const float d0 = a.adv[rix(a.idx, i)] - mean, d1 = a.adv[rix(a.idx, i + 256)] - mean;
        q0 += d0 * d0;
        q1 += d1 * d1;
    }
    if (i < a.n) {
        const float d0 = a.adv[rix(a.idx, i)] - mean;
        q0 += d0 * d0;
    }
    const float var = block_sum4(q0 + q1, red, tid) / (float)(a.n - 1);
    const float adv_std = sqrtf(var);

    const float inv = 1.0f / (float)a.n;
    const float ent_coef = a.ent_coef[0];
    const float d_ent_term = inv * (-ent_coef);
    float st_v[NSTAT] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const int r = r0 + j;
        if (r >= a.n) break;   // uniform over the wave; later rows are past n too
        const float mx = wave_max(l[j]);
        float e = on ? expf(l[j] - mx) : 0.f;
        const float sum = wave_sum(e);
        const float lse = mx + logf(sum);
        const float logp = on ? l[j] - lse : 0.f;
        const float p = on ? expf(logp) : 0.f;
        const float ent = -wave_sum(p * logp);
        const float lp_act = __shfl(logp, act[j], 64);
        const float adv_n = (adv[j] - mean) / (adv_std + 1e-8f);
        // value loss + gradient (pufferlib.cu:1068-1085)
        const float v_err = vpred[j] - vold[j];
        const float v_clipped = vold[j] + fmaxf(-a.vf_clip, fminf(a.vf_clip, v_err));
        const float vl_u = (vpred[j] - ret[j]) * (vpred[j] - ret[j]);
        const float vl_c = (v_clipped - ret[j]) * (v_clipped - ret[j]);
        const float v_loss = 0.5f * fmaxf(vl_u, vl_c);
        float d_v = 0.f;
        if (vl_c > vl_u) {
            if (v_err >= -a.vf_clip && v_err <= a.vf_clip) d_v = v_clipped - ret[j];
        } else {
            d_v = vpred[j] - ret[j];
        }
        // policy loss + gradient (pufferlib.cu:1133-1180)
        const float logratio = lp_act - old_logp[j];
        const float ratio = expf(logratio);
        const float rc = fmaxf(1.0f - a.clip, fminf(1.0f + a.clip, ratio));
        const float wa = -w[j] * adv_n;
        const float pg1 = wa * ratio, pg2 = wa * rc;
        const float pg = fmaxf(pg1, pg2);
        float d_ratio = wa * inv;
        if (pg2 > pg1 && (ratio <= 1.0f - a.clip || ratio >= 1.0f + a.clip)) d_ratio = 0.f;
        const float dnl = d_ratio * ratio;
        if (on) {
            float g = (lane == act[j]) ? dnl : 0.f;
            g -= p * dnl;
            g += d_ent_term * p * (-ent - logp);
            a.grad[(long)r * (A + 1) + lane] = g;
        }
        if (lane == 0) {
            a.grad[(long)r * (A + 1) + A] = inv * a.vf_coef * d_v;
            if (a.ratio) a.ratio[r] = ratio;
            if (a.newvalue) a.newvalue[r] = vpred[j];
        }
        st_v[0] += pg * inv;
        st_v[1] += v_loss * inv;
        st_v[2] += ent * inv;
        st_v[3] += (pg + a.vf_coef * v_loss - ent_coef * ent) * inv;
        st_v[4] += -logratio * inv;
        st_v[5] += ((ratio - 1.0f) - logratio) * inv;
        st_v[6] += (fabsf(ratio - 1.0f) > a.clip ? 1.0f : 0.0f) * inv;
    }
    if (lane == 0)
        for (int c = 0; c < NSTAT; ++c) rowstat[wave][c] = st_v[c];
    __syncthreads();
    if (tid < NSTAT)
        a.partial[(long)blockIdx.x * NSTAT + tid] =
            ((rowstat[0][tid] + rowstat[1][tid]) + rowstat[2][tid]) + rowstat[3][tid];
}

// fixed-order sums of the block partials, one wave per statistic (lane-
// strided, then the wave's butterfly); stats[0..6] += sums, stats[7] += 1;
// guard = (approx_kl, v_loss) of this minibatch (pufferlib.cu:1254-1284)
__global__ __launch_bounds__(64 * NSTAT) void ppo_reduce_kernel(const float* part, int blocks, float* stats,
                                                               float* guard) {
    const int c = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float s = 0.f;
    for (int b = lane; b < blocks; b += 64) s += part[(long)b * NSTAT + c];
    s = wave_sum(s);
    if (lane != 0) return;
    if (stats) {
        stats[c] += s;
        if (c == 0) stats[NSTAT] += 1.0f;
    }
    if (guard) {
        if (c == 5) guard[0] = s;
        if (c == 1) guard[1] = s;
    }
}

// pufferlib.cu:1292-1302: a threshold <= 0 disables its test, a non-finite
// value fails it; skipped[0] counts every veto, skipped[1] the vetoes whose
// value test failed (KL_GUARD_SKIPPED / KL_GUARD_SKIPPED_VF)
__global__ void kl_gate_kernel(const float* guard, float kl_thr, float vf_thr, float* gate,
                               float* skipped) {
    const float kl = guard[0], vf = guard[1];
    const bool kl_ok = (kl_thr <= 0.0f) || (isfinite(kl) && kl <= kl_thr);
    const bool vf_ok = (vf_thr <= 0.0f) || (isfinite(vf) && vf <= vf_thr);
    const float pass = (kl_ok && vf_ok) ? 1.0f : 0.0f;
    gate[0] = pass;
    if (skipped) {
        skipped[0] += 1.0f - pass;
        skipped[1] += vf_ok ? 0.0f : 1.0f;
    }
}

}  // namespace

long pt_ppo_partial_floats(int n) { return (long)pt_cdiv(n, RPB) * NSTAT; }

int pt_ppo_loss(const float* out, int n, int A, const float* mask, long mask_stride,
                const int32_t* idx, const float* actions, const float* old_logp,
                const float* adv, const float* ret, const float* val, const float* prio,
                float clip, float vf_clip, float vf_coef, const float* ent_coef, float* grad,
                float* ratio, float* newvalue, float* stats, float* guard, float* partial,
                hipStream_t s) {
    PT_REQUIRE(ent_coef != nullptr, "ppo loss: ent_coef must be a device scalar");
    PT_REQUIRE(n >= 2, "ppo loss: need at least 2 rows for the unbiased advantage variance (n=%d)", n);
    PT_REQUIRE(A >= 1 && A <= 64, "ppo loss: A=%d options unsupported (1..64)", A);
    PPOArgs a{out, n, A, mask, mask_stride, idx, actions, old_logp, adv, ret, val, prio,
              clip, vf_clip, vf_coef, ent_coef, grad, ratio, newvalue, partial};
    const int blocks = pt_cdiv(n, RPB);
    const int slot = pt_prof_open(s);
    hipLaunchKernelGGL(ppo_loss_kernel, dim3(blocks), dim3(256), 0, s, a);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(ppo_reduce_kernel, dim3(1), dim3(64 * NSTAT), 0, s, partial, blocks, stats, guard);
    PT_LAUNCH_CHECK();
    // algorithmic bytes per row: the (A+1) outputs and A mask floats read,
    // five per-row inputs (+ the importance weight), the (A+1) gradient and
    // ratio / new value written
    const double row_bytes = 4.0 * ((A + 1) + A + 5 + (prio ? 1 : 0) + (A + 1) + (ratio ? 1 : 0) + (newvalue ? 1 : 0));
    pt_prof_close(slot, PROF_PPO, n * row_bytes, s);
    return PTCG_OK;
}

int pt_kl_gate(const float* guard, float kl_thr, float vf_thr, float* gate, float* skipped,
               hipStream_t s) {
    hipLaunchKernelGGL(kl_gate_kernel, dim3(1), dim3(1), 0, s, guard, kl_thr, vf_thr, gate, skipped);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
