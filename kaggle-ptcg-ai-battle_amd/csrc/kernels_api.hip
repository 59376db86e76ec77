// extern "C" wrappers of the individual kernels (include/ptcg_amd_kernels.h).
#include "model.h"
#include "../../include/ptcg_amd_kernels.h"

extern "C" int ptcg_kernel_gemm(int M, int N, int K, const float* A, int64_t lda, int a_t,
                                const float* B, int64_t ldb, int b_t, float* C, int64_t ldc,
                                int epi, const float* bias, const float* R, int64_t ldr, float* C2,
                                int64_t ldc2, float* workspace, int64_t workspace_floats,
                                void* stream) {
    PT_REQUIRE(A && B && C, "kernel_gemm: null operand");
    PT_REQUIRE(epi >= EPI_STORE && epi <= EPI_MUL, "kernel_gemm: bad epilogue %d", epi);
    PT_REQUIRE(!((epi == EPI_BIAS || epi == EPI_BIAS_GELU || epi == EPI_BIAS_RESID || epi == EPI_BIAS_GELU_D) && !bias),
               "kernel_gemm: epilogue %d needs bias", epi);
    PT_REQUIRE(!((epi == EPI_BIAS_RESID || epi == EPI_GELU_BWD || epi == EPI_MUL) && !R),
               "kernel_gemm: epilogue %d needs R", epi);
    PT_REQUIRE(!((epi == EPI_BIAS_GELU || epi == EPI_BIAS_GELU_D) && !C2), "kernel_gemm: epilogue %d needs C2", epi);
    GemmArgs g{};
    g.M = M; g.N = N; g.K = K;
    g.A = A; g.lda = lda; g.a_t = a_t;
    g.B = B; g.ldb = ldb; g.b_t = b_t;
    g.C = C; g.ldc = ldc; g.epi = epi;
    g.bias = bias; g.R = R; g.ldr = ldr; g.C2 = C2; g.ldc2 = ldc2;
    return pt_gemm(g, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_rows_dev(int M, int N, int K, const float* A, int64_t lda, const float* B,
                                         int64_t ldb, int b_t, float* C, int64_t ldc, int epi, const float* bias,
                                         const float* R, int64_t ldr, float* C2, int64_t ldc2,
                                         const int* rows_dev, float* workspace, int64_t workspace_floats,
                                         void* stream) {
    PT_REQUIRE(rows_dev, "kernel_gemm_rows_dev: null device row count");
    PT_REQUIRE(A && B && C, "kernel_gemm_rows_dev: null operand");
    PT_REQUIRE(epi >= EPI_STORE && epi <= EPI_MUL, "kernel_gemm_rows_dev: bad epilogue %d", epi);
    PT_REQUIRE(!((epi == EPI_BIAS || epi == EPI_BIAS_GELU || epi == EPI_BIAS_RESID || epi == EPI_BIAS_GELU_D) && !bias),
               "kernel_gemm_rows_dev: epilogue %d needs bias", epi);
    PT_REQUIRE(!((epi == EPI_BIAS_RESID || epi == EPI_GELU_BWD || epi == EPI_MUL) && !R),
               "kernel_gemm_rows_dev: epilogue %d needs R", epi);
    PT_REQUIRE(!((epi == EPI_BIAS_GELU || epi == EPI_BIAS_GELU_D) && !C2),
               "kernel_gemm_rows_dev: epilogue %d needs C2", epi);
    GemmArgs g{};
    g.M = M; g.N = N; g.K = K;
    g.A = A; g.lda = lda; g.a_t = 0;
    g.B = B; g.ldb = ldb; g.b_t = b_t;
    g.C = C; g.ldc = ldc; g.epi = epi;
    g.bias = bias; g.R = R; g.ldr = ldr; g.C2 = C2; g.ldc2 = ldc2;
    g.Mdev = rows_dev;
    return pt_gemm(g, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_axpby(int M, int N, int K, const float* A, int64_t lda, int a_t,
                                      const float* B, int64_t ldb, int b_t, float* C, int64_t ldc, float alpha,
                                      const float* R, int64_t ldr, float beta, void* stream) {
    PT_REQUIRE(A && B && C && R, "kernel_gemm_axpby: null operand");
    GemmArgs g{};
    g.M = M; g.N = N; g.K = K;
    g.A = A; g.lda = lda; g.a_t = a_t;
    g.B = B; g.ldb = ldb; g.b_t = b_t;
    g.C = C; g.ldc = ldc; g.epi = EPI_AXPBY;
    g.R = R; g.ldr = ldr;
    g.alpha = alpha; g.beta = beta;
    return pt_gemm(g, nullptr, 0, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_bf16(int M, int N, int K, const float* A, int64_t lda, int a_t,
                                     const float* B, int64_t ldb, int b_t, float* C, int64_t ldc,
                                     int epi, const float* bias, const float* R, int64_t ldr, float* C2,
                                     int64_t ldc2, float* workspace, int64_t workspace_floats,
                                     void* stream) {
    PT_REQUIRE(A && B && C, "kernel_gemm_bf16: null operand");
    PT_REQUIRE(epi >= EPI_STORE && epi <= EPI_MUL, "kernel_gemm_bf16: bad epilogue %d", epi);
    GemmArgs g{};
    g.M = M; g.N = N; g.K = K;
    g.A = A; g.lda = lda; g.a_t = a_t;
    g.B = B; g.ldb = ldb; g.b_t = b_t;
    g.C = C; g.ldc = ldc; g.epi = epi;
    g.bias = bias; g.R = R; g.ldr = ldr; g.C2 = C2; g.ldc2 = ldc2;
    g.prec = 1;
    return pt_gemm(g, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_dw(int rows, int in, int out, const float* dY, int64_t lddy,
                                   const float* X, int64_t ldx, float* dW, float* db,
                                   float* workspace, int64_t workspace_floats, void* stream) {
    PT_REQUIRE(dY && X && dW, "kernel_gemm_dw: null operand");
    GemmArgs g{};
    g.M = out; g.N = in; g.K = rows;
    g.A = dY; g.lda = lddy; g.a_t = 1;
    g.B = X; g.ldb = ldx; g.b_t = 1;
    g.C = dW; g.ldc = in; g.epi = EPI_STORE;
    g.dbias = db;
    return pt_gemm(g, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_dw_rows_dev(int rows, int in, int out, const float* dY, int64_t lddy,
                                            const float* X, int64_t ldx, float* dW, float* db,
                                            const int* rows_dev, float* workspace, int64_t workspace_floats,
                                            void* stream) {
    PT_REQUIRE(dY && X && dW && rows_dev, "kernel_gemm_dw_rows_dev: null operand");
    GemmArgs g{};
    g.M = out; g.N = in; g.K = rows;
    g.A = dY; g.lda = lddy; g.a_t = 1;
    g.B = X; g.ldb = ldx; g.b_t = 1;
    g.C = dW; g.ldc = in; g.epi = EPI_STORE;
    g.dbias = db;
    g.Kdev = rows_dev;
    return pt_gemm(g, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_dw_bf16(int rows, int in, int out, const float* dY, int64_t lddy,
                                        const float* X, int64_t ldx, float* dW, float* db,
                                        float* workspace, int64_t workspace_floats, void* stream) {
    PT_REQUIRE(dY && X && dW, "kernel_gemm_dw_bf16: null operand");
    GemmArgs g{};
    g.M = out; g.N = in; g.K = rows;
    g.A = dY; g.lda = lddy; g.a_t = 1;
    g.B = X; g.ldb = ldx; g.b_t = 1;
    g.C = dW; g.ldc = in; g.epi = EPI_STORE;
    g.dbias = db;
    g.prec = 1;
    return pt_gemm(g, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_bs(int M, int N, int K, const void* A, int64_t lda, const void* B, int64_t ldb,
                                   void* C, int64_t ldc, int epi, int out_bf16, const float* bias, const void* R,
                                   int64_t ldr, void* C2, int64_t ldc2, void* stream) {
    PT_REQUIRE(A && B && C, "kernel_gemm_bs: null operand");
    PT_REQUIRE(!((epi == EPI_BIAS || epi == EPI_BIAS_RESID || epi == EPI_BIAS_GELU_D) && !bias),
               "kernel_gemm_bs: epilogue %d needs bias", epi);
    PT_REQUIRE(!((epi == EPI_BIAS_RESID || epi == EPI_MUL) && !R), "kernel_gemm_bs: epilogue %d needs R", epi);
    PT_REQUIRE(!(epi == EPI_BIAS_GELU_D && !C2), "kernel_gemm_bs: epilogue %d needs C2", epi);
    GemmArgs g{};
    g.M = M; g.N = N; g.K = K;
    g.A = (const float*)A; g.lda = lda;
    g.B = (const float*)B; g.ldb = ldb;
    g.C = (float*)C; g.ldc = ldc; g.epi = epi;
    g.bias = bias; g.R = (const float*)R; g.ldr = ldr; g.C2 = (float*)C2; g.ldc2 = ldc2;
    g.prec = 1; g.bs = 1; g.obf = out_bf16 != 0;
    return pt_gemm(g, nullptr, 0, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_dw_bs(int rows, int in, int out, const void* dY, int64_t lddy, const void* X,
                                      int64_t ldx, float* dW, float* db, float* workspace, int64_t workspace_floats,
                                      void* stream) {
    PT_REQUIRE(dY && X && dW, "kernel_gemm_dw_bs: null operand");
    GemmArgs g{};
    g.M = out; g.N = in; g.K = rows;
    g.A = (const float*)dY; g.lda = lddy; g.a_t = 1;
    g.B = (const float*)X; g.ldb = ldx; g.b_t = 1;
    g.C = dW; g.ldc = in; g.epi = EPI_STORE;
    g.dbias = db;
    g.prec = 1; g.bs = 1;
    return pt_gemm(g, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_colsum(const float* X, int64_t ldx, int M, int N, float* out,
                                  float* workspace, int64_t workspace_floats, void* stream) {
    PT_REQUIRE(X && out, "kernel_colsum: null buffer");
    return pt_colsum(X, ldx, M, N, out, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_layernorm_fwd(const float* x, const float* w, const float* b, float* y,
                                         float* mean, float* rstd, int rows, int D, void* stream) {
    PT_REQUIRE(x && w && b && y && mean && rstd, "kernel_layernorm_fwd: null buffer");
    return pt_ln_fwd(x, D, w, b, y, D, mean, rstd, rows, D, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_gemm_resid_ln(int rows, int K, const void* A, const void* W, const float* bias,
                                         const float* R, float* C, const float* lnw, const float* lnb, void* y,
                                         float* mean, float* rstd, int bf16, const int* rows_dev, void* stream) {
    PT_REQUIRE(rows > 0 && K > 0, "kernel_gemm_resid_ln: empty shape %d x %d", rows, K);
    GemmArgs g{};
    g.M = rows; g.N = 256; g.K = K;
    g.prec = bf16 ? 1 : 0; g.bs = bf16 ? 1 : 0;
    g.A = static_cast<const float*>(A); g.lda = K;
    g.B = static_cast<const float*>(W); g.ldb = K;
    g.C = C; g.ldc = 256;
    g.bias = bias; g.R = R; g.ldr = 256;
    g.epi = EPI_BIAS_RESID;
    g.Mdev = rows_dev;
    return pt_gemm_resid_ln(g, lnw, lnb, static_cast<float*>(y), 256, mean, rstd, (hipStream_t)stream, bf16);
}

extern "C" int ptcg_kernel_gemm_dx_layernorm_bwd(int rows, int K, const void* dY, const void* WT, const float* x,
                                                const float* w, const float* mean, const float* rstd,
                                                const float* dres, float* dx, void* dxh, float* dw, float* db,
                                                float* workspace, int64_t workspace_floats, const int* rows_dev,
                                                void* stream) {
    PT_REQUIRE(rows > 0 && K > 0, "kernel_gemm_dx_layernorm_bwd: empty shape %d x %d", rows, K);
    GemmArgs g{};
    g.M = rows; g.N = 256; g.K = K;
    g.prec = 1; g.bs = 1;
    g.A = static_cast<const float*>(dY); g.lda = K;
    g.B = static_cast<const float*>(WT); g.ldb = K;
    g.epi = EPI_STORE;
    g.Mdev = rows_dev;
    return pt_dx_lnbwd(g, x, w, mean, rstd, dres, dx, static_cast<float*>(dxh), dw, db, workspace,
                       workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_layernorm_bwd(const float* dy, const float* x, const float* w,
                                         const float* mean, const float* rstd, const float* dres,
                                         float* dx, float* dw, float* db, int rows, int D,
                                         float* workspace, int64_t workspace_floats, void* stream) {
    PT_REQUIRE(dy && x && w && mean && rstd && dx, "kernel_layernorm_bwd: null buffer");
    return pt_ln_bwd(dy, D, x, D, w, mean, rstd, dres, D, dx, D, dw, db, rows, D, workspace,
                     workspace_floats, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_attention_fwd(const float* qkv, const float* keep, float* ctx, float* lse,
                                         int N, int L, int H, int Dh, void* stream) {
    PT_REQUIRE(qkv && keep && ctx && lse, "kernel_attention_fwd: null buffer");
    return pt_attn_fwd(qkv, keep, ctx, lse, N, L, H, Dh, (hipStream_t)stream);
}

extern "C" int ptcg_kernel_attention_fwd_bf16(const float* qkv, const float* keep, float* ctx, float* lse,
                                              int N, int L, int H, int Dh, void* stream) {
    PT_REQUIRE(qkv && keep && ctx && lse, "kernel_attention_fwd_bf16: null buffer");
    return pt_attn_fwd(qkv, keep, ctx, lse, N, L, H, Dh, (hipStream_t)stream, nullptr, 1);
}

extern "C" int ptcg_kernel_attention_bwd_bf16(const float* qkv, const float* keep, const float* ctx,
                                              const float* lse, const float* dctx, float* dqkv, int N,
                                              int L, int H, int Dh, void* stream) {
    PT_REQUIRE(qkv && keep && ctx && lse && dctx && dqkv, "kernel_attention_bwd_bf16: null buffer");
    return pt_attn_bwd(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, Dh, (hipStream_t)stream, nullptr, 1);
}

extern "C" int64_t ptcg_kernel_attention_bwd_ws_bytes(int N, int L, int H, int Dh, int bf16) {
    return (int64_t)pt_attn_bwd_ws_bytes(N, L, H, Dh, bf16 ? 1 : 0);
}

extern "C" int ptcg_kernel_attention_bwd_ws(const float* qkv, const float* keep, const float* ctx,
                                            const float* lse, const float* dctx, float* dqkv, int N, int L,
                                            int H, int Dh, int bf16, void* workspace, int64_t workspace_bytes,
                                            void* stream) {
    PT_REQUIRE(qkv && keep && ctx && lse && dctx && dqkv, "kernel_attention_bwd_ws: null buffer");
    const size_t need = pt_attn_bwd_ws_bytes(N, L, H, Dh, bf16 ? 1 : 0);
    PT_REQUIRE(need > 0, "kernel_attention_bwd_ws: L=%d Dh=%d takes the recompute pair (no dS scratch)", L, Dh);
    PT_REQUIRE(workspace && workspace_bytes >= (int64_t)need,
               "kernel_attention_bwd_ws: workspace of %lld bytes, need %zu", (long long)workspace_bytes, need);
    return pt_attn_bwd(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, Dh, (hipStream_t)stream, nullptr, bf16 ? 1 : 0,
                       workspace, (size_t)workspace_bytes);
}

int pt_attn_path(int L, int DH);
extern "C" int ptcg_kernel_attention_path(int L, int Dh) { return pt_attn_path(L, Dh); }

extern "C" int ptcg_kernel_attention_bwd(const float* qkv, const float* keep, const float* ctx,
                                         const float* lse, const float* dctx, float* dqkv, int N,
                                         int L, int H, int Dh, void* stream) {
    PT_REQUIRE(qkv && keep && ctx && lse && dctx && dqkv, "kernel_attention_bwd: null buffer");
    return pt_attn_bwd(qkv, keep, ctx, lse, dctx, dqkv, N, L, H, Dh, (hipStream_t)stream);
}
