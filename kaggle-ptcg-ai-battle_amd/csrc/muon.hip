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
// is M x N with M <= N, zero-padded to multiples of 16; per-matrix
// normalisation), one launch applies every matrix update, and each
// Newton-Schulz phase is ONE grouped GEMM launch over all matrices' tiles
// (the LDS-DMA MFMA kernel; the Gram products split K and a grouped
// fixed-order reduce sums them; the alpha / beta epilogue forms b A + c A A
// and a X + B X).  The padding keeps every product on the DMA tile rules and
// stays exactly zero through the iteration.  A step is ~30 launches where
// the reference issues ~20 per matrix; the grads are read, never written
// (the reference clips and transforms them in place).
#include "model.h"
#include "../../include/ptcg_amd.h"

namespace {

constexpr int MU_NT = 256;
constexpr int MU_EPB = 4;                 // elements per thread in the segment kernels
constexpr int MU_CHUNK = MU_NT * MU_EPB;  // elements per workgroup
constexpr int MU_NPART = 512;             // clip partials
constexpr int MU_NT_NORM = 512;
constexpr int MU_PAD = 16;                // canonical matrices padded to multiples of 16

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
    int Mp, Np;     // padded to multiples of 16
    int tall;       // R > C: the canonical matrix is X^T
    int p0;         // first of this matrix's norm partials (one per canonical chunk)
    float scale;    // sqrt(max(1, R/C))
};

// chunk -> (segment, first element); matrices' chunks run over the padded
// canonical positions (momentum, normalisation) or over their own elements
// (update)
struct MuonChunk {
    int seg;
    int start;
};

// source element of canonical position (i, j) of a matrix
__device__ __forceinline__ long src_of(const MuonSeg& s, int i, int j) {
    return s.tall ? (long)j * s.C + i : (long)i * s.C + j;
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

// momentum for every tensor; vectors finish here, matrices write their
// Nesterov output to the padded canonical layout (zeros in the padding) and
// one sum-of-squares partial per chunk
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
    if (s.C == 0) {
#pragma unroll
        for (int k = 0; k < MU_EPB; ++k) {
            const long e = (long)ch.start + k * MU_NT + threadIdx.x;
            if (e >= s.n) break;
            const long i = s.off + e;
            const float gc = g[i] * coef;
            const float m = mu * mom[i] + (1.0f - mu) * gc;
            mom[i] = m;
            const float u = gc + m;
            w[i] = w[i] * (1.0f - lr * wd_1d) - lr * 1.0f * u;
        }
        return;
    }
    const long total = (long)s.Mp * s.Np;
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < MU_EPB; ++k) {
        const long q = (long)ch.start + k * MU_NT + threadIdx.x;
        if (q >= total) break;
        const int ci = (int)(q / s.Np), cj = (int)(q % s.Np);
        float u = 0.f;
        if (ci < s.M && cj < s.N) {
            const long i = s.off + src_of(s, ci, cj);
            const float gc = g[i] * coef;
            const float m = mu * mom[i] + gc;
            mom[i] = m;
            u = gc + mu * m;
            sq += u * u;
        }
        Y[s.y + q] = u;
    }
    __shared__ float red[MU_NT / 64];
    sq = wave_sum(sq);
    __syncthreads();   // clip_coef's reduction array is separate; keep the stages apart
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
    __syncthreads();
    if (threadIdx.x == 0) ypart[s.p0 + ch.start / MU_CHUNK] = ((red[0] + red[1]) + red[2]) + red[3];
}

// X = u / max(||u||_F, 1e-7) for every matrix (canonical chunks)
__global__ __launch_bounds__(MU_NT) void muon_normalize_kernel(const MuonSeg* __restrict__ segs,
                                                              const MuonChunk* __restrict__ chunks,
                                                              float* __restrict__ Y, const float* __restrict__ ypart,
                                                              const float* __restrict__ gate) {
    if (gate && gate[0] == 0.0f) return;
    const MuonChunk ch = chunks[blockIdx.x];
    const MuonSeg s = segs[ch.seg];
    const long total = (long)s.Mp * s.Np;
    const int np = (int)((total + MU_CHUNK - 1) / MU_CHUNK);
    float t = 0.f;
    for (int p = 0; p < np; ++p) t += ypart[s.p0 + p];
    const float inv = 1.0f / fmaxf(sqrtf(t), 1e-7f);
#pragma unroll
    for (int k = 0; k < MU_EPB; ++k) {
        const long q = (long)ch.start + k * MU_NT + threadIdx.x;
        if (q >= total) break;
        Y[s.y + q] *= inv;
    }
}

// w = w (1 - lr wd) - lr scale X for every matrix (chunks of its elements)
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
        const int r = (int)(e / s.C), c = (int)(e % s.C);
        const long q = s.tall ? (long)c * s.Np + r : (long)r * s.Np + c;
        const long i = s.off + e;
        w[i] = w[i] * wd_scale - lr * s.scale * Y[s.y + q];
    }
}

// one phase of a Newton-Schulz iteration: a grouped launch over all matrices
struct NsPhase {
    GroupedGemm* d = nullptr;     // device descriptors
    int* d_items = nullptr;       // work item -> descriptor
    int items = 0, count = 0;
    int* d_rchunk = nullptr;      // reduce chunk -> descriptor (split-K phases)
    int* d_rfirst = nullptr;      // descriptor -> first reduce chunk
    int rchunks = 0;
    int a_t = 0, b_t = 0, epi = EPI_STORE, partial = 0;
    double flops = 0.0;           // 2 M N K of the unpadded products
};

}  // namespace

struct PtcgMuon {
    PtcgDims dm{};
    long arena = 0;
    float momentum = 0.f, wd = 0.f, wd_1d = 0.f;
    std::vector<MuonSeg> segs;
    int n_all_chunks = 0, n_can_chunks = 0, n_src_chunks = 0, n_ypart = 0;
    char* mem = nullptr;
    MuonSeg* d_segs = nullptr;
    MuonChunk* d_all = nullptr;   // vectors' element chunks + matrices' canonical chunks
    MuonChunk* d_can = nullptr;   // matrices' canonical chunks
    MuonChunk* d_src = nullptr;   // matrices' element chunks
    float *mom = nullptr, *Y0 = nullptr, *Y1 = nullptr, *Ga = nullptr, *Gb = nullptr, *Gp = nullptr;
    float *part = nullptr, *ypart = nullptr, *lr = nullptr;
    NsPhase ns[5][4];             // per iteration: Gram (split K + reduce), polynomial, update wide, update tall
    double ns_flops = 0.0;        // Newton-Schulz products per step (unpadded shapes)
};

namespace {

// descriptors of one phase: upload them and the work-item map into mem at `at`
struct PhaseBuild {
    std::vector<GroupedGemm> gs;
    std::vector<int> items, rchunk, rfirst;
};

void phase_add(PhaseBuild& pb, const GemmArgs& g, int splits, int k_chunk, long part_stride, float* out) {
    GroupedGemm d{};
    d.g = g;
    d.splits = splits;
    d.k_chunk = k_chunk;
    d.part_stride = part_stride;
    d.out = out;
    d.tiles = pt_cdiv(g.M, 128) * pt_cdiv(g.N, 128);
    d.first = (int)pb.items.size();
    const int gi = (int)pb.gs.size();
    for (int w = 0; w < d.tiles * splits; ++w) pb.items.push_back(gi);
    if (out) {
        pb.rfirst.push_back((int)pb.rchunk.size());
        const long tot = (long)g.M * g.N;
        for (long c = 0; c < tot; c += 1024) pb.rchunk.push_back(gi);
    } else {
        pb.rfirst.push_back(0);
    }
    pb.gs.push_back(d);
}

}  // namespace

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
    long off = 0, y = 0, gfl = 0, gpart = 0;
    std::vector<MuonChunk> all, can, src;
    std::vector<long> g_off, gp_off;
    std::vector<int> splits_of, kchunk_of;
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
        const int seg = (int)m->segs.size();
        if (s.C > 0) {
            s.M = std::min(s.R, s.C);
            s.N = std::max(s.R, s.C);
            s.Mp = (s.M + MU_PAD - 1) / MU_PAD * MU_PAD;
            s.Np = (s.N + MU_PAD - 1) / MU_PAD * MU_PAD;
            s.tall = s.R > s.C;
            s.y = y;
            const long can_n = (long)s.Mp * s.Np;
            y += can_n;
            s.p0 = p0;
            p0 += (int)((can_n + MU_CHUNK - 1) / MU_CHUNK);
            s.scale = sqrtf(fmaxf(1.0f, (float)s.R / (float)s.C));
            // Gram split: chunks of >= 128 along K, at most 16
            int sp = std::max(1, std::min(16, s.Np / 128));
            const int kc = pt_cdiv(pt_cdiv(s.Np, sp), 16) * 16;
            sp = pt_cdiv(s.Np, kc);
            g_off.push_back(gfl);
            gp_off.push_back(gpart);
            splits_of.push_back(sp);
            kchunk_of.push_back(kc);
            gfl += (long)s.Mp * s.Mp;
            gpart += (long)sp * s.Mp * s.Mp;
            m->ns_flops += 5.0 * (4.0 * s.M * (double)s.M * s.N + 2.0 * s.M * (double)s.M * s.M);
            for (long c = 0; c < can_n; c += MU_CHUNK) {
                all.push_back(MuonChunk{seg, (int)c});
                can.push_back(MuonChunk{seg, (int)c});
            }
            for (long c = 0; c < s.n; c += MU_CHUNK) src.push_back(MuonChunk{seg, (int)c});
        } else {
            g_off.push_back(-1);
            gp_off.push_back(-1);
            splits_of.push_back(0);
            kchunk_of.push_back(0);
            for (long c = 0; c < s.n; c += MU_CHUNK) all.push_back(MuonChunk{seg, (int)c});
        }
        m->segs.push_back(s);
        off += s.n;
    }
    m->arena = ptcg_arena_floats(dims);
    PT_REQUIRE(((off + 3) & ~3L) == m->arena, "muon_create: arena walk %ld != arena %ld", off, m->arena);
    m->n_all_chunks = (int)all.size();
    m->n_can_chunks = (int)can.size();
    m->n_src_chunks = (int)src.size();
    m->n_ypart = p0;

    size_t total = 0;
    auto take = [&](size_t bytes) { total = (total + 255) & ~(size_t)255; size_t o = total; total += bytes; return o; };
    const size_t oSeg = take(m->segs.size() * sizeof(MuonSeg)), oAll = take(all.size() * sizeof(MuonChunk)),
                 oCan = take(std::max<size_t>(1, can.size()) * sizeof(MuonChunk)),
                 oSrc = take(std::max<size_t>(1, src.size()) * sizeof(MuonChunk)), oMom = take(m->arena * 4),
                 oY0 = take(std::max(1L, y) * 4), oY1 = take(std::max(1L, y) * 4), oGa = take(std::max(1L, gfl) * 4),
                 oGb = take(std::max(1L, gfl) * 4), oGp = take(std::max(1L, gpart) * 4), oPart = take(MU_NPART * 4),
                 oYp = take(std::max(1, p0) * 4), oLr = take(4);
    // Newton-Schulz phase descriptors (pointers into this allocation: built
    // after the base address is known)
    const size_t fixed = total;
    (void)fixed;
    PhaseBuild pb[5][4];
    size_t oPh[5][4][5];
    for (int it = 0; it < 5; ++it)
        for (int ph = 0; ph < 4; ++ph) {
            // sizes first (pointer values filled below): count descriptors and items
            PhaseBuild& b = pb[it][ph];
            for (size_t i = 0; i < m->segs.size(); ++i) {
                const MuonSeg& sg = m->segs[i];
                if (sg.C == 0) continue;
                if (ph == 3 && !sg.tall) continue;
                if (ph == 2 && sg.tall) continue;
                GemmArgs g{};
                g.M = sg.Mp;
                g.N = ph >= 2 ? sg.Np : sg.Mp;
                phase_add(b, g, ph == 0 ? splits_of[i] : 1, 0, 0, ph == 0 ? (float*)1 : nullptr);
            }
            oPh[it][ph][0] = take(std::max<size_t>(1, b.gs.size()) * sizeof(GroupedGemm));
            oPh[it][ph][1] = take(std::max<size_t>(1, b.items.size()) * sizeof(int));
            oPh[it][ph][2] = take(std::max<size_t>(1, b.rchunk.size()) * sizeof(int));
            oPh[it][ph][3] = take(std::max<size_t>(1, b.rfirst.size()) * sizeof(int));
        }
    hipError_t e = hipMalloc(&m->mem, total);
    if (e != hipSuccess) {
        ptcg_set_error("muon_create: hipMalloc(%zu): %s", total, hipGetErrorString(e));
        delete m;
        return PTCG_ERR_HIP;
    }
    m->d_segs = (MuonSeg*)(m->mem + oSeg);
    m->d_all = (MuonChunk*)(m->mem + oAll);
    m->d_can = (MuonChunk*)(m->mem + oCan);
    m->d_src = (MuonChunk*)(m->mem + oSrc);
    m->mom = (float*)(m->mem + oMom);
    m->Y0 = (float*)(m->mem + oY0);
    m->Y1 = (float*)(m->mem + oY1);
    m->Ga = (float*)(m->mem + oGa);
    m->Gb = (float*)(m->mem + oGb);
    m->Gp = (float*)(m->mem + oGp);
    m->part = (float*)(m->mem + oPart);
    m->ypart = (float*)(m->mem + oYp);
    m->lr = (float*)(m->mem + oLr);
    // the phases' descriptors with real pointers
    for (int it = 0; it < 5; ++it) {
        float* X = (it % 2 == 0) ? m->Y0 : m->Y1;
        float* Xn = (it % 2 == 0) ? m->Y1 : m->Y0;
        const float a = NS_COEF[it][0], b = NS_COEF[it][1], c = NS_COEF[it][2];
        for (int ph = 0; ph < 4; ++ph) {
            PhaseBuild nb;
            for (size_t i = 0; i < m->segs.size(); ++i) {
                const MuonSeg& sg = m->segs[i];
                if (sg.C == 0) continue;
                if (ph == 3 && !sg.tall) continue;
                if (ph == 2 && sg.tall) continue;
                const int Mp = sg.Mp, Np = sg.Np;
                float* x = X + sg.y;
                float* xn = Xn + sg.y;
                float* A = m->Ga + g_off[i];
                float* B = m->Gb + g_off[i];
                GemmArgs g{};
                if (ph == 0) {   // A = X X^T: split-K partials, reduced into A
                    g.M = Mp; g.N = Mp; g.K = Np;
                    g.A = x; g.lda = Np; g.a_t = 0;
                    g.B = x; g.ldb = Np; g.b_t = 0;
                    g.C = m->Gp + gp_off[i]; g.ldc = Mp; g.epi = EPI_STORE;
                    phase_add(nb, g, splits_of[i], kchunk_of[i], (long)Mp * Mp, A);
                } else if (ph == 1) {   // B = c A A + b A
                    g.M = Mp; g.N = Mp; g.K = Mp;
                    g.A = A; g.lda = Mp; g.a_t = 0;
                    g.B = A; g.ldb = Mp; g.b_t = 1;
                    g.C = B; g.ldc = Mp; g.epi = EPI_AXPBY;
                    g.R = A; g.ldr = Mp; g.alpha = c; g.beta = b;
                    phase_add(nb, g, 1, Mp, 0, nullptr);
                } else {   // X' = a X + B X; a tall matrix's X B is (B^T X^T)^T: B read transposed
                    g.M = Mp; g.N = Np; g.K = Mp;
                    g.A = B; g.lda = Mp; g.a_t = sg.tall;
                    g.B = x; g.ldb = Np; g.b_t = 1;
                    g.C = xn; g.ldc = Np; g.epi = EPI_AXPBY;
                    g.R = x; g.ldr = Np; g.alpha = 1.0f; g.beta = a;
                    phase_add(nb, g, 1, Mp, 0, nullptr);
                }
            }
            NsPhase& P = m->ns[it][ph];
            for (size_t i = 0; i < m->segs.size(); ++i) {
                const MuonSeg& sg = m->segs[i];
                if (sg.C == 0 || (ph == 3 && !sg.tall) || (ph == 2 && sg.tall)) continue;
                P.flops += ph == 0 ? 2.0 * sg.M * (double)sg.M * sg.N
                                   : ph == 1 ? 2.0 * sg.M * (double)sg.M * sg.M : 2.0 * sg.M * (double)sg.N * sg.M;
            }
            P.count = (int)nb.gs.size();
            P.items = (int)nb.items.size();
            P.rchunks = ph == 0 ? (int)nb.rchunk.size() : 0;
            P.a_t = ph == 3 ? 1 : 0;
            P.b_t = ph == 0 ? 0 : 1;
            P.epi = ph == 0 ? EPI_STORE : EPI_AXPBY;
            P.partial = ph == 0;
            P.d = (GroupedGemm*)(m->mem + oPh[it][ph][0]);
            P.d_items = (int*)(m->mem + oPh[it][ph][1]);
            P.d_rchunk = (int*)(m->mem + oPh[it][ph][2]);
            P.d_rfirst = (int*)(m->mem + oPh[it][ph][3]);
            if (P.count == 0) continue;
            if (hipMemcpy(P.d, nb.gs.data(), nb.gs.size() * sizeof(GroupedGemm), hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(P.d_items, nb.items.data(), nb.items.size() * sizeof(int), hipMemcpyHostToDevice) != hipSuccess ||
                (ph == 0 && (hipMemcpy(P.d_rchunk, nb.rchunk.data(), nb.rchunk.size() * sizeof(int),
                                       hipMemcpyHostToDevice) != hipSuccess ||
                             hipMemcpy(P.d_rfirst, nb.rfirst.data(), nb.rfirst.size() * sizeof(int),
                                       hipMemcpyHostToDevice) != hipSuccess))) {
                ptcg_set_error("muon_create: descriptor upload failed");
                ptcg_muon_free(m);
                return PTCG_ERR_HIP;
            }
        }
    }
    // momentum and workspaces start at zero (muon_post_create :205-213)
    if (hipMemset(m->mom, 0, (size_t)(oGp - oMom) + (size_t)std::max(1L, gpart) * 4) != hipSuccess ||
        hipMemcpy(m->d_segs, m->segs.data(), m->segs.size() * sizeof(MuonSeg), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->d_all, all.data(), all.size() * sizeof(MuonChunk), hipMemcpyHostToDevice) != hipSuccess ||
        (!can.empty() &&
         hipMemcpy(m->d_can, can.data(), can.size() * sizeof(MuonChunk), hipMemcpyHostToDevice) != hipSuccess) ||
        (!src.empty() &&
         hipMemcpy(m->d_src, src.data(), src.size() * sizeof(MuonChunk), hipMemcpyHostToDevice) != hipSuccess)) {
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

// the learning rate the update kernels read (device float), synchronous
int pt_muon_lr(PtcgMuon* m, float* lr) {
    PT_REQUIRE(m && lr, "muon_lr: null argument");
    PT_HIP(hipMemcpy(lr, m->lr, 4, hipMemcpyDeviceToHost));
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
    const int slot = pt_prof_open(s);
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
    if (m->n_can_chunks > 0) {
        hipLaunchKernelGGL(muon_normalize_kernel, dim3(m->n_can_chunks), dim3(MU_NT), 0, s, m->d_segs, m->d_can,
                           m->Y0, m->ypart, gate);
        PT_LAUNCH_CHECK();
        // Newton-Schulz: the padded canonical X ping-pongs between Y0 and Y1
        const int prev_class = pt_prof_gemm_class(PROF_MUON_GEMM);
        int r = PTCG_OK;
        for (int it = 0; it < 5 && r == PTCG_OK; ++it)
            for (int ph = 0; ph < 4 && r == PTCG_OK; ++ph) {
                const NsPhase& P = m->ns[it][ph];
                if (P.count == 0) continue;
                r = pt_gemm_grouped(P.d, P.d_items, P.items, P.a_t, P.b_t, P.epi, P.partial, P.flops, s);
                if (r == PTCG_OK && P.rchunks > 0) r = pt_grouped_reduce(P.d, P.d_rchunk, P.d_rfirst, P.rchunks, s);
            }
        pt_prof_gemm_class(prev_class);
        PT_TRY(r);
        // after 5 iterations the result is in Y1
        hipLaunchKernelGGL(muon_update_kernel, dim3(m->n_src_chunks), dim3(MU_NT), 0, s, m->d_segs, m->d_src,
                           weights, m->Y1, m->wd, m->lr, gate);
        PT_LAUNCH_CHECK();
    }
    pt_prof_close(slot, PROF_MUON, m->ns_flops, s);
    return PTCG_OK;
}
