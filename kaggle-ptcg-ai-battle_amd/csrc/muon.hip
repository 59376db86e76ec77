// Muon over the flat fp32 parameter arena: global-norm clip, Nesterov
// momentum and Newton-Schulz orthogonalisation for matrices, EMA momentum and
// decoupled weight decay for vectors, gated like the trainer's KL guard.
//
// Replaces muon_init / muon_post_create / muon_step (native/src/muon.cu:
// 154-297) with the same arithmetic:
//   g' = g * min(max_norm / (||g||_2 + 1e-6), 1)            (:226-232, :107-114)
//   >= 2-D tensor (R x C):  m = mu m + g';  u = g' + mu m    (muon_nesterov :49-61)
//     X = u / max(||u||_F, 1e-7)                            (:250-255, :40-47)
//     5 x  A = X X^T (wide) / X^T X (tall);  B = c A A + b A;
//          X = a X + B X (wide) / a X + X B (tall)          (:257-282, ns_coeffs :116-122)
//     w = w (1 - lr wd) - lr sqrt(max(1, R/C)) X            (muon_weight_update :88-105)
//   1-D tensor:  m = mu m + (1 - mu) g';  w = w (1 - lr wd_1d) - lr (g' + m)
//                                                           (muon_nesterov_ema :63-86)
// A gate that reads 0 leaves weights and momentum untouched (:49-105).
//
// Layout for MI355X: the elementwise work is three launches over the whole
// arena (clip sums; momentum + vector updates + the matrices' Nesterov
// output written in a canonical wide layout, Y = X or X^T so every matrix
// is M x N with M <= N; per-matrix normalisation), the Newton-Schulz
// products run on the MFMA GEMM (split-K for the long Gram reductions, the
// alpha / beta epilogue for b A + c A A and a X + B X), and one launch
// applies every matrix update.  The reference issues ~20 launches per matrix
// and clips the grads in place; here the grads are read, never written.
#include "model.h"
#include "../../include/ptcg_amd.h"

namespace {

constexpr int MU_NT = 256;
constexpr int MU_EPB = 4;                 // elements per thread in the segment kernels
constexpr int MU_CHUNK = MU_NT * MU_EPB;  // elements per workgroup
constexpr int MU_NPART = 512;             // clip partials
constexpr int MU_NT_NORM = 512;

// Newton-Schulz quintic coefficients (a, b, c) per iteration (muon.cu:116-122)
constexpr float NS_COEF[5][3] = {
    {4.0848f, -6.8946f, 2.9270f}, {3.9505f, -6.3029f, 2.6377f}, {3.7418f, -5.5913f, 2.3037f},
    {2.8769f, -3.1427f, 1.2046f}, {2.8366f, -3.0525f, 1.2012f},
};

struct MuonSeg {
    long off;       // arena offset of the tensor
    long n;         // elements
    long y;         // canonical-layout offset (matrices), -1 for vectors
    int R, C;       // registered shape (C = 0: vector)
    int M, N;       // canonical: min / max of R, C
    int tall;       // R > C: the canonical matrix is X^T
    int p0;         // first of this matrix's norm partials (one per chunk)
    float scale;    // sqrt(max(1, R/C))
};

// chunk -> (segment, first element)
struct MuonChunk {
    int seg;
    int start;
};

__device__ __forceinline__ long canon(const MuonSeg& s, long e) {
    if (!s.tall) return e;
    const long r = e / s.C, c = e % s.C;
    return c * s.R + r;
}

__global__ __launch_bounds__(MU_NT_NORM) void muon_sumsq_kernel(const float4* __restrict__ g, long n4,
                                                                 const float* __restrict__ gate,
                                                                 float* __restrict__ part) {
    if (gate && gate[0] == 0.0f) return;
    __shared__ float red[MU_NT_NORM / 64];
    float s0 = 0.f, s1 = 0.f;
    const long stride = (long)gridDim.x * MU_NT_NORM;
    long i = (long)blockIdx.x * MU_NT_NORM + threadIdx.x;
    for (; i + stride < n4; i += 2 * stride) {
        const float4 a = g[i], b = g[i + stride];
        s0 += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
        s1 += (b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w);
    }
    if (i < n4) {
        const float4 a = g[i];
        s0 += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
    }
    const float s = wave_sum(s0 + s1);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < MU_NT_NORM / 64; ++w) t += red[w];
        part[blockIdx.x] = t;
    }
}

// every workgroup folds the clip partials in the same order
__device__ __forceinline__ float clip_coef(const float* part, int nparts, float max_norm, float* norm_out) {
    __shared__ float red[MU_NT / 64];
    float s = 0.f;
    for (int i = threadIdx.x; i < nparts; i += MU_NT) s += part[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float norm = sqrtf(((red[0] + red[1]) + red[2]) + red[3]);
    if (norm_out && blockIdx.x == 0 && threadIdx.x == 0) norm_out[0] = norm;
    return fminf(max_norm / (norm + 1e-6f), 1.0f);
}

// momentum for every tensor; vectors finish here, matrices leave their
// Nesterov output in the canonical layout plus one sum-of-squares partial
// per chunk
__global__ __launch_bounds__(MU_NT) void muon_momentum_kernel(
        const MuonSeg* __restrict__ segs, const MuonChunk* __restrict__ chunks, float* __restrict__ w,
        const float* __restrict__ g, float* __restrict__ mom, float* __restrict__ Y, float* __restrict__ ypart,
        const float* __restrict__ part, int nparts, float max_norm, float mu, float wd_1d,
        const float* __restrict__ lr_ptr, const float* __restrict__ gate, float* __restrict__ norm_out) {
    if (gate && gate[0] == 0.0f) return;
    const float coef = clip_coef(part, nparts, max_norm, norm_out);
    const MuonChunk ch = chunks[blockIdx.x];
    const MuonSeg s = segs[ch.seg];
    const float lr = *lr_ptr;
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < MU_EPB; ++k) {
        const long e = (long)ch.start + k * MU_NT + threadIdx.x;
        if (e >= s.n) break;
        const long i = s.off + e;
        const float gc = g[i] * coef;
        if (s.C == 0) {
            const float m = mu * mom[i] + (1.0f - mu) * gc;
            mom[i] = m;
            const float u = gc + m;
            w[i] = w[i] * (1.0f - lr * wd_1d) - lr * 1.0f * u;
        } else {
            const float m = mu * mom[i] + gc;
            mom[i] = m;
            const float u = gc + mu * m;
            Y[s.y + canon(s, e)] = u;
            sq += u * u;
        }
    }
    if (s.C != 0) {
        __shared__ float red[MU_NT / 64];
        sq = wave_sum(sq);
        __syncthreads();   // red of clip_coef is a different array; keep the stages apart
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
        __syncthreads();
        if (threadIdx.x == 0) ypart[s.p0 + ch.start / MU_CHUNK] = ((red[0] + red[1]) + red[2]) + red[3];
    }
}

// X = u / max(||u||_F, 1e-7) for every matrix (chunks of matrices only)
__global__ __launch_bounds__(MU_NT) void muon_normalize_kernel(const MuonSeg* __restrict__ segs,
                                                              const MuonChunk* __restrict__ chunks,
                                                              float* __restrict__ Y, const float* __restrict__ ypart,
                                                              const float* __restrict__ gate) {
    if (gate && gate[0] == 0.0f) return;
    const MuonChunk ch = chunks[blockIdx.x];
    const MuonSeg s = segs[ch.seg];
    const int np = (int)((s.n + MU_CHUNK - 1) / MU_CHUNK);
    float t = 0.f;
    for (int p = 0; p < np; ++p) t += ypart[s.p0 + p];
    const float inv = 1.0f / fmaxf(sqrtf(t), 1e-7f);
#pragma unroll
    for (int k = 0; k < MU_EPB; ++k) {
        const long e = (long)ch.start + k * MU_NT + threadIdx.x;
        if (e >= s.n) break;
        Y[s.y + e] *= inv;
    }
}

// w = w (1 - lr wd) - lr scale X for every matrix (chunks of matrices only)
__global__ __launch_bounds__(MU_NT) void muon_update_kernel(const MuonSeg* __restrict__ segs,
                                                           const MuonChunk* __restrict__ chunks,
                                                           float* __restrict__ w, const float* __restrict__ Y,
                                                           float wd, const float* __restrict__ lr_ptr,
                                                           const float* __restrict__ gate) {
    if (gate && gate[0] == 0.0f) return;
    const MuonChunk ch = chunks[blockIdx.x];
    const MuonSeg s = segs[ch.seg];
    const float lr = *lr_ptr;
    const float wd_scale = 1.0f - lr * wd;
#pragma unroll
    for (int k = 0; k < MU_EPB; ++k) {
        const long e = (long)ch.start + k * MU_NT + threadIdx.x;
        if (e >= s.n) break;
        const long i = s.off + e;
        w[i] = w[i] * wd_scale - lr * s.scale * Y[s.y + canon(s, e)];
    }
}

}  // namespace

struct PtcgMuon {
    PtcgDims dm{};
    long arena = 0;
    float momentum = 0.f, wd = 0.f, wd_1d = 0.f;
    std::vector<MuonSeg> segs;
    int n_all_chunks = 0, n_mat_chunks = 0, n_ypart = 0;
    long y_floats = 0, g_floats = 0, ws_floats = 0;
    char* mem = nullptr;
    MuonSeg* d_segs = nullptr;
    MuonChunk* d_all = nullptr;   // every tensor's chunks
    MuonChunk* d_mat = nullptr;   // matrices' chunks
    float *mom = nullptr, *Y0 = nullptr, *Y1 = nullptr, *Ga = nullptr, *Gb = nullptr, *ws = nullptr;
    float *part = nullptr, *ypart = nullptr, *lr = nullptr;
    std::vector<long> g_off;      // per matrix segment: Gram workspace offset (M x M)
};

extern "C" void ptcg_muon_free(PtcgMuon* m) {
    if (!m) return;
    if (m->mem) (void)hipFree(m->mem);
    delete m;
}

extern "C" int ptcg_muon_create(const PtcgDims* dims, double lr, double momentum, double weight_decay,
                                double wd_1d, PtcgMuon** out) {
    PT_REQUIRE(dims && out, "muon_create: null argument");
    std::vector<ParamDef> defs(512);
    const int np = pt_param_table(*dims, defs.data(), (int)defs.size());
    PT_REQUIRE(np > 0, "muon_create: bad dims");
    PtcgMuon* m = new PtcgMuon();
    m->dm = *dims;
    m->momentum = (float)momentum;
    m->wd = (float)weight_decay;
    m->wd_1d = (float)wd_1d;
    // the arena walk of muon_step (:236-245): tensor starts rounded up to 4 floats
    long off = 0, y = 0, gfl = 0, maxMM = 0;
    std::vector<MuonChunk> all, mat;
    int p0 = 0;
    for (int i = 0; i < np; ++i) {
        const ParamDef& d = defs[i];
        off = (off + 3) & ~3L;
        MuonSeg s{};
        s.off = off;
        s.n = d.rows * (d.cols > 0 ? d.cols : 1);
        s.R = (int)d.rows;
        s.C = d.cols > 0 ? (int)d.cols : 0;
        s.y = -1;
        if (s.C > 0) {
            s.M = std::min(s.R, s.C);
            s.N = std::max(s.R, s.C);
            s.tall = s.R > s.C;
            s.y = y;
            y += (s.n + 3) & ~3L;
            s.p0 = p0;
            p0 += (int)((s.n + MU_CHUNK - 1) / MU_CHUNK);
            s.scale = sqrtf(fmaxf(1.0f, (float)s.R / (float)s.C));
            m->g_off.push_back(gfl);
            gfl += ((long)s.M * s.M + 3) & ~3L;
            maxMM = std::max(maxMM, (long)s.M * s.M);
        } else {
            m->g_off.push_back(-1);
        }
        const int seg = (int)m->segs.size();
        for (long c = 0; c < s.n; c += MU_CHUNK) {
            all.push_back(MuonChunk{seg, (int)c});
            if (s.C > 0) mat.push_back(MuonChunk{seg, (int)c});
        }
        m->segs.push_back(s);
        off += s.n;
    }
    m->arena = ptcg_arena_floats(dims);
    PT_REQUIRE(((off + 3) & ~3L) == m->arena, "muon_create: arena walk %ld != arena %ld", off, m->arena);
    m->n_all_chunks = (int)all.size();
    m->n_mat_chunks = (int)mat.size();
    m->n_ypart = p0;
    m->y_floats = y;
    m->g_floats = gfl;
    m->ws_floats = std::max(8L << 20, 64 * maxMM);
    size_t total = 0;
    auto take = [&](size_t bytes) { total = (total + 255) & ~(size_t)255; size_t o = total; total += bytes; return o; };
    const size_t oSeg = take(m->segs.size() * sizeof(MuonSeg)), oAll = take(all.size() * sizeof(MuonChunk)),
                 oMat = take(std::max<size_t>(1, mat.size()) * sizeof(MuonChunk)), oMom = take(m->arena * 4),
                 oY0 = take(std::max(1L, y) * 4), oY1 = take(std::max(1L, y) * 4), oGa = take(std::max(1L, gfl) * 4),
                 oGb = take(std::max(1L, gfl) * 4), oWs = take(m->ws_floats * 4), oPart = take(MU_NPART * 4),
                 oYp = take(std::max(1, p0) * 4), oLr = take(4);
    hipError_t e = hipMalloc(&m->mem, total);
    if (e != hipSuccess) {
        ptcg_set_error("muon_create: hipMalloc(%zu): %s", total, hipGetErrorString(e));
        delete m;
        return PTCG_ERR_HIP;
    }
    m->d_segs = (MuonSeg*)(m->mem + oSeg);
    m->d_all = (MuonChunk*)(m->mem + oAll);
    m->d_mat = (MuonChunk*)(m->mem + oMat);
    m->mom = (float*)(m->mem + oMom);
    m->Y0 = (float*)(m->mem + oY0);
    m->Y1 = (float*)(m->mem + oY1);
    m->Ga = (float*)(m->mem + oGa);
    m->Gb = (float*)(m->mem + oGb);
    m->ws = (float*)(m->mem + oWs);
    m->part = (float*)(m->mem + oPart);
    m->ypart = (float*)(m->mem + oYp);
    m->lr = (float*)(m->mem + oLr);
    // momentum and workspaces start at zero (muon_post_create :205-213)
    if (hipMemset(m->mem, 0, total) != hipSuccess ||
        hipMemcpy(m->d_segs, m->segs.data(), m->segs.size() * sizeof(MuonSeg), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->d_all, all.data(), all.size() * sizeof(MuonChunk), hipMemcpyHostToDevice) != hipSuccess ||
        (!mat.empty() &&
         hipMemcpy(m->d_mat, mat.data(), mat.size() * sizeof(MuonChunk), hipMemcpyHostToDevice) != hipSuccess)) {
        ptcg_set_error("muon_create: device upload failed");
        ptcg_muon_free(m);
        return PTCG_ERR_HIP;
    }
    const float lr_f = (float)lr;
    if (hipMemcpy(m->lr, &lr_f, 4, hipMemcpyHostToDevice) != hipSuccess) {
        ptcg_set_error("muon_create: lr upload failed");
        ptcg_muon_free(m);
        return PTCG_ERR_HIP;
    }
    *out = m;
    return PTCG_OK;
}

extern "C" int ptcg_muon_set_lr(PtcgMuon* m, float lr) {
    PT_REQUIRE(m, "muon_set_lr: null optimizer");
    PT_HIP(hipMemcpy(m->lr, &lr, 4, hipMemcpyHostToDevice));
    return PTCG_OK;
}

extern "C" float* ptcg_muon_momentum(PtcgMuon* m) { return m ? m->mom : nullptr; }

int pt_muon_set_momentum(PtcgMuon* m, double momentum) {
    PT_REQUIRE(m, "muon: null optimizer");
    m->momentum = (float)momentum;
    return PTCG_OK;
}

extern "C" int ptcg_muon_step(PtcgMuon* m, float* weights, const float* grads, float max_grad_norm,
                              const float* gate, float* grad_norm_out, void* stream) {
    PT_REQUIRE(m && weights && grads, "muon_step: null argument");
    PT_REQUIRE((((uintptr_t)weights | (uintptr_t)grads) & 15) == 0, "muon_step: arenas must be 16 B aligned");
    hipStream_t s = (hipStream_t)stream;
    const long n4 = m->arena / 4;
    int parts = pt_cdiv(n4, MU_NT_NORM * 2);
    if (parts > MU_NPART) parts = MU_NPART;
    hipLaunchKernelGGL(muon_sumsq_kernel, dim3(parts), dim3(MU_NT_NORM), 0, s, (const float4*)grads, n4, gate,
                       m->part);
    PT_LAUNCH_CHECK();
    hipLaunchKernelGGL(muon_momentum_kernel, dim3(m->n_all_chunks), dim3(MU_NT), 0, s, m->d_segs, m->d_all, weights,
                       grads, m->mom, m->Y0, m->ypart, m->part, parts, max_grad_norm, m->momentum, m->wd_1d, m->lr,
                       gate, grad_norm_out);
    PT_LAUNCH_CHECK();
    if (m->n_mat_chunks == 0) return PTCG_OK;
    hipLaunchKernelGGL(muon_normalize_kernel, dim3(m->n_mat_chunks), dim3(MU_NT), 0, s, m->d_segs, m->d_mat, m->Y0,
                       m->ypart, gate);
    PT_LAUNCH_CHECK();
    // Newton-Schulz: canonical X (M x N, M <= N) ping-pongs between Y0 and Y1
    for (int it = 0; it < 5; ++it) {
        float* X = (it % 2 == 0) ? m->Y0 : m->Y1;
        float* Xn = (it % 2 == 0) ? m->Y1 : m->Y0;
        const float a = NS_COEF[it][0], b = NS_COEF[it][1], c = NS_COEF[it][2];
        for (size_t i = 0; i < m->segs.size(); ++i) {
            const MuonSeg& sg = m->segs[i];
            if (sg.C == 0) continue;
            const int M = sg.M, N = sg.N;
            float* x = X + sg.y;
            float* xn = Xn + sg.y;
            float* A = m->Ga + m->g_off[i];
            float* B = m->Gb + m->g_off[i];
            // A = X X^T
            GemmArgs g1{};
            g1.M = M; g1.N = M; g1.K = N;
            g1.A = x; g1.lda = N; g1.a_t = 0;
            g1.B = x; g1.ldb = N; g1.b_t = 0;
            g1.C = A; g1.ldc = M; g1.epi = EPI_STORE;
            PT_TRY(pt_gemm(g1, m->ws, m->ws_floats, s));
            // B = c A A + b A
            GemmArgs g2{};
            g2.M = M; g2.N = M; g2.K = M;
            g2.A = A; g2.lda = M; g2.a_t = 0;
            g2.B = A; g2.ldb = M; g2.b_t = 1;
            g2.C = B; g2.ldc = M; g2.epi = EPI_AXPBY;
            g2.R = A; g2.ldr = M; g2.alpha = c; g2.beta = b;
            PT_TRY(pt_gemm(g2, nullptr, 0, s));
            // X' = a X + B X in the canonical layout; for a tall matrix the
            // reference's X B is (B^T X^T)^T, so the product reads B transposed
            GemmArgs g3{};
            g3.M = M; g3.N = N; g3.K = M;
            g3.A = B; g3.lda = M; g3.a_t = sg.tall;
            g3.B = x; g3.ldb = N; g3.b_t = 1;
            g3.C = xn; g3.ldc = N; g3.epi = EPI_AXPBY;
            g3.R = x; g3.ldr = N; g3.alpha = 1.0f; g3.beta = a;
            PT_TRY(pt_gemm(g3, nullptr, 0, s));
        }
    }
    // after 5 iterations the result is in Y1
    hipLaunchKernelGGL(muon_update_kernel, dim3(m->n_mat_chunks), dim3(MU_NT), 0, s, m->d_segs, m->d_mat, weights,
                       m->Y1, m->wd, m->lr, gate);
    PT_LAUNCH_CHECK();
    return PTCG_OK;
}
