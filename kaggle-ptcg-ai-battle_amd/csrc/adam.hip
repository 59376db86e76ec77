// Fused global-norm clip + Adam over the flat fp32 parameter arena.
//
// Fills the optimizer slot of the reference trainer (muon_step,
// native/src/muon.cu:209-297, whose clip is muon_norm_partials /
// muon_norm_reduce / muon_clip_norm :3-46,107-114) with two launches:
//   1. sum-of-squares partials of the grad arena (128-bit loads, four in
//      flight per thread); block 0 also publishes the step number this call
//      will use;
//   2. persistent workgroups stride over chunks of the arena; every thread
//      issues the loads of its first chunk's p, g, m, v float4s, then its
//      workgroup folds the partials in the same fixed order (so all agree bit
//      for bit on ||g||) while those loads are in flight, and each chunk's
//      loads are issued before the previous chunk's stores; per element:
//      g' = g * min(max_norm / (||g|| + 1e-6), 1)
//      m  = m + (1 - b1) (g' - m);  v = v b2 + (1 - b2) g'^2
//      p  = p - (lr / (1 - b1^t)) m / (sqrt(v) / sqrt(1 - b2^t) + eps)
//      (torch.optim.Adam's single-tensor arithmetic: lerp_, mul_/addcmul_,
//      addcdiv_).  Thread 0 of workgroup 0 commits the step counter.
// The learning rate is read from a device double (the reference's lr_ptr,
// muon.cu:92-100), so a captured step follows the host's schedule writes.
// A device gate (the trainer's KL/value guard, pufferlib.cu:1292-1302) that
// reads 0 makes both launches return before touching memory, and the step
// counter does not advance: a vetoed step is a bit-exact no-op.
// Gap floats of the 16 B-aligned arena have g = 0, so they stay 0.
// HBM traffic: 4 B/param (pass 1) + 28 B/param (pass 2: read p,g,m,v,
// write p,m,v).
#include "common.h"

namespace {

constexpr int NPART = 512;    // pass-1 workgroups (upper bound) = norm partials
constexpr int NT_NORM = 512;
constexpr int NT = 256;
constexpr int UPD_U = 2;      // float4s per thread and chunk in pass 2, loaded together
// pass-2 workgroups (persistent, striding over the chunks): four per CU.
// Measured per update over 4.3 M parameters by launch events (nontemporal
// streams): 24.9 us at 1024 x (U = 2), 25.8 at 768, 26.2 at 512, 26.2 at 2048;
// U = 1 with 1024 or 2048 blocks 25.7 / 26.9; U = 4 with 512 / 256 blocks
// 28.6 / 32.1
constexpr int UPD_BLOCKS = 1024;

// streaming loads / stores of the update (nontemporal: none of p, g, m, v is
// read again in this launch; 26.7 -> 25.9 us per update by launch events)
typedef float ntfx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ntl(const float4* p) {
    const ntfx4 v = __builtin_nontemporal_load(reinterpret_cast<const ntfx4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void nts(float4 v, float4* p) {
    const ntfx4 x = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(x, reinterpret_cast<ntfx4*>(p));
}
__device__ __forceinline__ float sq4(float4 v) { return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w); }

__global__ __launch_bounds__(NT_NORM) void adam_norm_kernel(const float4* __restrict__ g, long n4,
        const float* __restrict__ gate, const int32_t* __restrict__ step,
        float* __restrict__ ws) {
    if (gate && gate[0] == 0.0f) return;
    __shared__ float red[NT_NORM / 64];
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    const long stride = (long)gridDim.x * NT_NORM;
    long i = (long)blockIdx.x * NT_NORM + threadIdx.x;
    for (; i + 3 * stride < n4; i += 4 * stride) {
        const float4 a = g[i], b = g[i + stride], c = g[i + 2 * stride], d = g[i + 3 * stride];
        s0 += sq4(a);
        s1 += sq4(b);
        s2 += sq4(c);
        s3 += sq4(d);
    }
    for (; i < n4; i += stride) s0 += sq4(g[i]);
    const float s = wave_sum((s0 + s1) + (s2 + s3));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < NT_NORM / 64; ++w) t += red[w];
        ws[blockIdx.x] = t;
        // the step this update applies: previous count + 1
        if (blockIdx.x == 0) reinterpret_cast<int32_t*>(ws + NPART)[0] = step[0] + 1;
    }
}

// LR: the learning rate's device type (double: the trainer's scalar; float:
// the reference trainer's lr_ptr), widened to double before use
template <int U, typename LR>
__global__ __launch_bounds__(NT) void adam_update_kernel(float4* __restrict__ p,
        const float4* __restrict__ g, float4* __restrict__ m, float4* __restrict__ v, long n4,
        int nparts, const LR* __restrict__ lr_dev, double b1, double b2, double eps, float max_norm,
        const float* __restrict__ gate, const float* __restrict__ ws, float* __restrict__ norm_out,
        int32_t* __restrict__ step) {
    if (gate && gate[0] == 0.0f) return;
    // persistent: workgroup b takes chunks b, b + G, ... (G = gridDim.x) of
    // NT * U float4s; a chunk's loads are issued before the previous chunk's
    // stores, so reads and writes stream together
    const long stride = (long)gridDim.x * (NT * U);
    long base = (long)blockIdx.x * (NT * U) + threadIdx.x;
    float4 gg[U], mm[U], vv[U], pp[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long i = base + (long)u * NT;
        if (i < n4) {
            gg[u] = ntl(g + i);
            mm[u] = ntl(m + i);
            vv[u] = ntl(v + i);
            pp[u] = ntl(p + i);
        }
    }
    __shared__ float red[NT / 64];
    float s = 0.f;
    for (int i = threadIdx.x; i < nparts; i += NT) s += ws[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float norm = sqrtf(((red[0] + red[1]) + red[2]) + red[3]);
    const float coef = fminf(max_norm / (norm + 1e-6f), 1.0f);
    const int t = reinterpret_cast<const int32_t*>(ws + NPART)[0];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        if (norm_out) norm_out[0] = norm;
        step[0] = t;
    }
    // scalars in double, rounded once to fp32 (torch keeps them as Python
    // floats and hands fp32 kernels the rounded value)
    const double lr = (double)lr_dev[0];
    const float step_size = (float)(lr / (1.0 - pow(b1, (double)t)));
    const float bc2s = (float)sqrt(1.0 - pow(b2, (double)t));
    const float omb1 = (float)(1.0 - b1), omb2 = (float)(1.0 - b2);
    const float b2f = (float)b2, epsf = (float)eps;
    for (; base < n4; base += stride) {
        float4 g2[U], m2[U], v2[U], p2[U];
        const long nb = base + stride;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long i = nb + (long)u * NT;
            if (i < n4) {
                g2[u] = ntl(g + i);
                m2[u] = ntl(m + i);
                v2[u] = ntl(v + i);
                p2[u] = ntl(p + i);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long i = base + (long)u * NT;
            if (i < n4) {
#define PT_ADAM_LANE(c)                                             \
                {                                                   \
                    const float gc = gg[u].c * coef;                \
                    mm[u].c = mm[u].c + omb1 * (gc - mm[u].c);      \
                    vv[u].c = vv[u].c * b2f + omb2 * gc * gc;       \
                    const float den = sqrtf(vv[u].c) / bc2s + epsf; \
                    pp[u].c = pp[u].c + (-step_size) * (mm[u].c / den); \
                }
                PT_ADAM_LANE(x) PT_ADAM_LANE(y) PT_ADAM_LANE(z) PT_ADAM_LANE(w)
#undef PT_ADAM_LANE
                nts(mm[u], m + i);
                nts(vv[u], v + i);
                nts(pp[u], p + i);
            }
            gg[u] = g2[u];
            mm[u] = m2[u];
            vv[u] = v2[u];
            pp[u] = p2[u];
        }
    }
}

}  // namespace

long pt_adam_ws_floats() { return NPART + 4; }

template <typename LR>
static int adam_step(float* w, float* g, float* m, float* v, long n, const LR* lr, double b1, double b2,
                     double eps, float max_norm, const float* gate, int32_t* step, float* norm_out,
                     float* ws, hipStream_t s) {
    PT_REQUIRE(lr != nullptr, "adam: the learning rate must be a device scalar");
    PT_REQUIRE(n > 0 && n % 4 == 0, "adam: arena length %ld must be a positive multiple of 4", n);
    PT_REQUIRE(((uintptr_t)w | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) % 16 == 0,
               "adam: arenas must be 16 B aligned");
    PT_REQUIRE(ws != nullptr && step != nullptr, "adam: workspace and step counter required");
    const long n4 = n / 4;
    int parts = pt_cdiv(n4, NT_NORM * 4);
    if (parts > NPART) parts = NPART;
    if (parts < 1) parts = 1;
    int slot = pt_prof_open(s);
    hipLaunchKernelGGL(adam_norm_kernel, dim3(parts), dim3(NT_NORM), 0, s, (const float4*)g, n4, gate, step, ws);
    PT_LAUNCH_CHECK();
    pt_prof_close(slot, PROF_ADAM_NORM, 4.0 * n, s);
    long ublocks = (n4 + NT * UPD_U - 1) / (NT * UPD_U);
    if (ublocks > UPD_BLOCKS) ublocks = UPD_BLOCKS;
    slot = pt_prof_open(s);
    hipLaunchKernelGGL((adam_update_kernel<UPD_U, LR>), dim3((unsigned)ublocks), dim3(NT), 0, s, (float4*)w,
                       (const float4*)g, (float4*)m, (float4*)v, n4, parts, lr, b1, b2, eps, max_norm, gate, ws,
                       norm_out, step);
    PT_LAUNCH_CHECK();
    pt_prof_close(slot, PROF_ADAM_UPDATE, 28.0 * n, s);
    return PTCG_OK;
}

int pt_adam_step(float* w, float* g, float* m, float* v, long n, const double* lr, double b1, double b2,
                 double eps, float max_norm, const float* gate, int32_t* step, float* norm_out,
                 float* ws, hipStream_t s) {
    return adam_step(w, g, m, v, n, lr, b1, b2, eps, max_norm, gate, step, norm_out, ws, s);
}

int pt_adam_step(float* w, float* g, float* m, float* v, long n, const float* lr, double b1, double b2,
                 double eps, float max_norm, const float* gate, int32_t* step, float* norm_out,
                 float* ws, hipStream_t s) {
    return adam_step(w, g, m, v, n, lr, b1, b2, eps, max_norm, gate, step, norm_out, ws, s);
}
