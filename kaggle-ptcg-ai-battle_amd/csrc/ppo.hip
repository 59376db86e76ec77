// PPO clipped-surrogate + clipped value + entropy loss, forward statistics
// and hand-written gradient, for one discrete head of A <= 64 options.
//
// Same formulas as the reference's ppo_var_mean / ppo_discrete_head /
// ppo_loss_compute / ppo_loss_reduce (native/src/pufferlib.cu:949-1363),
// T_seq = 1 and no league tag: advantage normalised per minibatch with the
// unbiased variance, mask == 0 -> logit -1e4, ratio = exp(logp - old_logp),
// pg = max(-w adv_n r, -w adv_n clip(r)), v_loss = 0.5 max((v-R)^2,
// (v_old + clip(v - v_old) - R)^2), everything / N.  Layout differs: one
// wave64 per row with lane = option (the reference runs one thread per row
// over a serial 64-option loop), and the advantage statistics are computed
// redundantly by every workgroup in the same fixed order instead of by a
// separate <<<1,256>>> kernel, so the step is two launches.
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

__global__ __launch_bounds__(256) void ppo_loss_kernel(PPOArgs a) {
    __shared__ float red[256];
    __shared__ float red2[256];
    __shared__ float rowstat[4][NSTAT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // minibatch advantage mean / unbiased variance (pufferlib.cu:1307-1363)
    float s = 0.f;
    for (int i = tid; i < a.n; i += 256) s += a.adv[rix(a.idx, i)];
    red[tid] = s;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) red[tid] += red[tid + st];
        __syncthreads();
    }
    const float mean = red[0] / (float)a.n;
    float q = 0.f;
    for (int i = tid; i < a.n; i += 256) {
        float dd = a.adv[rix(a.idx, i)] - mean;
        q += dd * dd;
    }
    red2[tid] = q;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) red2[tid] += red2[tid + st];
        __syncthreads();
    }
    const float var = red2[0] / (float)(a.n - 1);
    const float adv_std = sqrtf(var);

    const int r = blockIdx.x * 4 + wave;
    float st_v[NSTAT] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (r < a.n) {
        const int src = rix(a.idx, r);
        const int A = a.A;
        const float inv = 1.0f / (float)a.n;
        const float* lg = a.out + (long)r * (A + 1);
        const float* mk = a.mask + (long)src * a.mask_stride;
        const bool on = lane < A;
        float l = -INFINITY;
        if (on) l = (mk[lane] == 0.f) ? -1e4f : lg[lane];
        const float mx = wave_max(l);
        float e = on ? expf(l - mx) : 0.f;
        const float sum = wave_sum(e);
        const float lse = mx + logf(sum);
        const float logp = on ? l - lse : 0.f;
        const float p = on ? expf(logp) : 0.f;
        const float ent = -wave_sum(p * logp);
        const int act = (int)a.actions[src];
        const float lp_act = __shfl(logp, act, 64);

        const float old_logp = a.old_logp[src];
        const float adv = a.adv[src];
        const float w = a.prio ? a.prio[src] : 1.0f;
        const float vold = a.val[src];
        const float ret = a.ret[src];
        const float vpred = lg[A];
        const float adv_n = (adv - mean) / (adv_std + 1e-8f);

        const float ent_coef = a.ent_coef[0];
        const float d_ent_term = inv * (-ent_coef);
        // value loss + gradient (pufferlib.cu:1068-1085)
        const float v_err = vpred - vold;
        const float v_clipped = vold + fmaxf(-a.vf_clip, fminf(a.vf_clip, v_err));
        const float vl_u = (vpred - ret) * (vpred - ret);
        const float vl_c = (v_clipped - ret) * (v_clipped - ret);
        const float v_loss = 0.5f * fmaxf(vl_u, vl_c);
        float d_v = 0.f;
        if (vl_c > vl_u) {
            if (v_err >= -a.vf_clip && v_err <= a.vf_clip) d_v = v_clipped - ret;
        } else {
            d_v = vpred - ret;
        }
        // policy loss + gradient (pufferlib.cu:1133-1180)
        const float logratio = lp_act - old_logp;
        const float ratio = expf(logratio);
        const float rc = fmaxf(1.0f - a.clip, fminf(1.0f + a.clip, ratio));
        const float wa = -w * adv_n;
        const float pg1 = wa * ratio, pg2 = wa * rc;
        const float pg = fmaxf(pg1, pg2);
        float d_ratio = wa * inv;
        if (pg2 > pg1 && (ratio <= 1.0f - a.clip || ratio >= 1.0f + a.clip)) d_ratio = 0.f;
        const float dnl = d_ratio * ratio;
        if (on) {
            float g = (lane == act) ? dnl : 0.f;
            g -= p * dnl;
            g += d_ent_term * p * (-ent - logp);
            a.grad[(long)r * (A + 1) + lane] = g;
        }
        if (lane == 0) {
            a.grad[(long)r * (A + 1) + A] = inv * a.vf_coef * d_v;
            if (a.ratio) a.ratio[r] = ratio;
            if (a.newvalue) a.newvalue[r] = vpred;
        }
        st_v[0] = pg * inv;
        st_v[1] = v_loss * inv;
        st_v[2] = ent * inv;
        st_v[3] = (pg + a.vf_coef * v_loss - ent_coef * ent) * inv;
        st_v[4] = -logratio * inv;
        st_v[5] = ((ratio - 1.0f) - logratio) * inv;
        st_v[6] = (fabsf(ratio - 1.0f) > a.clip ? 1.0f : 0.0f) * inv;
    }
    if (lane == 0)
        for (int c = 0; c < NSTAT; ++c) rowstat[wave][c] = st_v[c];
    __syncthreads();
    if (tid < NSTAT)
        a.partial[(long)blockIdx.x * NSTAT + tid] =
            ((rowstat[0][tid] + rowstat[1][tid]) + rowstat[2][tid]) + rowstat[3][tid];
}

// fixed-order sum of the block partials; stats[0..6] += sums, stats[7] += 1;
// guard = (approx_kl, v_loss) of this minibatch (pufferlib.cu:1254-1284)
__global__ void ppo_reduce_kernel(const float* part, int blocks, float* stats, float* guard) {
    const int c = threadIdx.x;
    if (c > NSTAT) return;
    if (c == NSTAT) {
        if (stats) stats[NSTAT] += 1.0f;
        return;
    }
    float s = 0.f;
    for (int b = 0; b < blocks; ++b) s += part[(long)b * NSTAT + c];
    if (stats) stats[c] += s;
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

long pt_ppo_partial_floats(int n) { return (long)pt_cdiv(n, 4) * NSTAT; }

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
    const int blocks = pt_cdiv(n, 4);
    const int slot = pt_prof_open(s);
    hipLaunchKernelGGL(ppo_loss_kernel, dim3(blocks), dim3(256), 0, s, a);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(ppo_reduce_kernel, dim3(1), dim3(64), 0, s, partial, blocks, stats, guard);
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
