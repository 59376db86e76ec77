// Fused global-norm clip + Adam over the flat fp32 parameter arena.
//
// Fills the optimizer slot of the reference trainer (muon_step,
// native/src/muon.cu:209-297, whose clip is muon_norm_partials /
// muon_norm_reduce / muon_clip_norm :3-46,107-114) with two launches:
//   1. sum-of-squares partials of the grad arena (128-bit loads, grid-stride);
//      block 0 also publishes the step number this call will use;
//   2. every workgroup folds the partials in the same fixed order (so all
//      agree bit for bit on ||g||), then streams p, g, m, v once:
//      g' = g * min(max_norm / (||g|| + 1e-6), 1)
//      m  = m + (1 - b1) (g' - m);  v = v b2 + (1 - b2) g'^2
//      p  = p - (lr / (1 - b1^t)) m / (sqrt(v) / sqrt(1 - b2^t) + eps)
//      (torch.optim.Adam's single-tensor arithmetic: lerp_, mul_/addcmul_,
//      addcdiv_).
// A device gate (the trainer's KL/value guard, pufferlib.cu:1292-1302) that
// reads 0 makes both launches return before touching memory, and the step
// counter does not advance: a vetoed step is a bit-exact no-op.
// Gap floats of the 16 B-aligned arena have g = 0, so they stay 0.
// HBM traffic: 4 B/param (pass 1) + 28 B/param (pass 2: read p,g,m,v,
// write p,m,v).
#include "common.h"

namespace {

constexpr int NPART = 1024;   // pass-1 workgroups (upper bound)
constexpr int NT = 256;

__global__ __launch_bounds__(NT) void adam_norm_kernel(const float4* __restrict__ g, long n4,
        const float* __restrict__ gate, const int32_t* __restrict__ step,
        float* __restrict__ ws) {
    if (gate && gate[0] == 0.0f) return;
    __shared__ float red[NT];
    float s = 0.f;
    for (long i = (long)blockIdx.x * NT + threadIdx.x; i < n4; i += (long)gridDim.x * NT) {
        const float4 v = g[i];
        s += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int st = NT / 2; st > 0; st >>= 1) {
        if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        ws[blockIdx.x] = red[0];
        if (blockIdx.x == 0) {
            // the step this update applies: previous count + 1
            reinterpret_cast<int32_t*>(ws + NPART)[0] = step[0] + 1;
        }
    }
}

__global__ __launch_bounds__(NT) void adam_update_kernel(float4* __restrict__ p,
        const float4* __restrict__ g, float4* __restrict__ m, float4* __restrict__ v, long n4,
        int nparts, double lr, double b1, double b2, double eps, float max_norm,
        const float* __restrict__ gate, const float* __restrict__ ws, float* __restrict__ norm_out) {
    if (gate && gate[0] == 0.0f) return;
    __shared__ float red[NT];
    __shared__ float sh_coef;
    float s = 0.f;
    for (int i = threadIdx.x; i < nparts; i += NT) s += ws[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int st = NT / 2; st > 0; st >>= 1) {
        if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float norm = sqrtf(red[0]);
        sh_coef = fminf(max_norm / (norm + 1e-6f), 1.0f);
        if (blockIdx.x == 0 && norm_out) norm_out[0] = norm;
    }
    __syncthreads();
    const float coef = sh_coef;
    const int t = reinterpret_cast<const int32_t*>(ws + NPART)[0];
    // scalars in double, rounded once to fp32 (torch keeps them as Python
    // floats and hands fp32 kernels the rounded value)
    const float step_size = (float)(lr / (1.0 - pow(b1, (double)t)));
    const float bc2s = (float)sqrt(1.0 - pow(b2, (double)t));
    const float omb1 = (float)(1.0 - b1), omb2 = (float)(1.0 - b2);
    const float b2f = (float)b2, epsf = (float)eps;
    for (long i = (long)blockIdx.x * NT + threadIdx.x; i < n4; i += (long)gridDim.x * NT) {
        float4 gg = g[i], mm = m[i], vv = v[i], pp = p[i];
#define PT_ADAM_LANE(c)                                             \
        {                                                           \
            const float gc = gg.c * coef;                           \
            mm.c = mm.c + omb1 * (gc - mm.c);                       \
            vv.c = vv.c * b2f + omb2 * gc * gc;                     \
            const float den = sqrtf(vv.c) / bc2s + epsf;            \
            pp.c = pp.c + (-step_size) * (mm.c / den);              \
        }
        PT_ADAM_LANE(x) PT_ADAM_LANE(y) PT_ADAM_LANE(z) PT_ADAM_LANE(w)
#undef PT_ADAM_LANE
        m[i] = mm;
        v[i] = vv;
        p[i] = pp;
    }
}

__global__ void adam_step_commit_kernel(const float* gate, int32_t* step, const float* ws) {
    if (gate && gate[0] == 0.0f) return;
    step[0] = reinterpret_cast<const int32_t*>(ws + NPART)[0];
}

}  // namespace

long pt_adam_ws_floats() { return NPART + 4; }

int pt_adam_step(float* w, float* g, float* m, float* v, long n, double lr, double b1, double b2,
                 double eps, float max_norm, const float* gate, int32_t* step, float* norm_out,
                 float* ws, hipStream_t s) {
    PT_REQUIRE(n > 0 && n % 4 == 0, "adam: arena length %ld must be a positive multiple of 4", n);
    PT_REQUIRE(((uintptr_t)w | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) % 16 == 0,
               "adam: arenas must be 16 B aligned");
    PT_REQUIRE(ws != nullptr && step != nullptr, "adam: workspace and step counter required");
    const long n4 = n / 4;
    int parts = pt_cdiv(n4, NT * 4);
    if (parts > NPART) parts = NPART;
    if (parts < 1) parts = 1;
    hipLaunchKernelGGL(adam_norm_kernel, dim3(parts), dim3(NT), 0, s, (const float4*)g, n4, gate, step, ws);
    PT_LAUNCH_CHECK();
    int ublocks = pt_cdiv(n4, NT * 2);
    if (ublocks > 4096) ublocks = 4096;
    hipLaunchKernelGGL(adam_update_kernel, dim3(ublocks), dim3(NT), 0, s, (float4*)w, (const float4*)g,
                       (float4*)m, (float4*)v, n4, parts, lr, b1, b2, eps, max_norm, gate, ws, norm_out);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(adam_step_commit_kernel, dim3(1), dim3(1), 0, s, gate, step, ws);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
