/*
 * ptcg_amd_kernels.h — kernel-level C ABI of libptcg_amd.so.
 *
 * The building blocks the model driver is made of, exported one by one so a
 * caller (or a parity test) can run each on device buffers of its own.  All
 * pointers are device pointers; stream is a hipStream_t (NULL = null stream);
 * return 0 on success, negative on failure (message: ptcg_last_error()).
 * Reference counterparts are cited per entry point.
 */
#ifndef PTCG_AMD_KERNELS_H
#define PTCG_AMD_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* C[M,N] = epi(sum_k A(m,k) B(k,n)); A(m,k) = a_t ? A[k*lda+m] : A[m*lda+k],
 * B(k,n) = b_t ? B[k*ldb+n] : B[n*ldb+k].  epi: 0 store, 1 +bias[n],
 * 2 +bias then C2 = gelu(C), 3 +bias +R[m*ldr+n], 4 *= gelu'(R[m*ldr+n]),
 * 5 C += acc, 6 z = acc + bias[n], C = gelu'(z), C2 = gelu(z),
 * 7 C = acc * R[m*ldr+n] (6 and 7 are a GELU layer's forward / backward
 * keeping gelu'(z) instead of z).  workspace (may be NULL) enables split-K
 * for long K.
 * Replaces pt_gemm / pt_linear / pt_linear_bwd (ptcg_kernels.cuh:42-108).  */
int ptcg_kernel_gemm(int M, int N, int K, const float* A, int64_t lda, int a_t,
                     const float* B, int64_t ldb, int b_t, float* C, int64_t ldc, int epi,
                     const float* bias, const float* R, int64_t ldr, float* C2, int64_t ldc2,
                     float* workspace, int64_t workspace_floats, void* stream);

/* ptcg_kernel_gemm with a device row count, as the sync-free model's
 * launches run: M is the host's row bound, *rows_dev (device int, <= M) the
 * rows computed; rows past it are left alone.  A row-major A (a_t = 0) only;
 * no split-K; with B not transposed, a bound of S to 8 S tiles on S CUs
 * balances the last wave from the device count (the host-count launch's
 * tiles, K splits and partial sums).
 * No reference counterpart: the sync-free layout's own launch form.        */
int ptcg_kernel_gemm_rows_dev(int M, int N, int K, const float* A, int64_t lda, const float* B,
                              int64_t ldb, int b_t, float* C, int64_t ldc, int epi, const float* bias,
                              const float* R, int64_t ldr, float* C2, int64_t ldc2, const int* rows_dev,
                              float* workspace, int64_t workspace_floats, void* stream);

/* C = alpha * op(A) op(B) + beta * R (R may not alias C), the alpha / beta
 * form of cublasGemmExDense / puf_addmm_nn (native/src/kernels.cu:262-310)
 * that the reference's Muon Newton-Schulz steps use (muon.cu:270-282);
 * operand conventions as ptcg_kernel_gemm.                                 */
int ptcg_kernel_gemm_axpby(int M, int N, int K, const float* A, int64_t lda, int a_t,
                           const float* B, int64_t ldb, int b_t, float* C, int64_t ldc, float alpha,
                           const float* R, int64_t ldr, float beta, void* stream);

/* ptcg_kernel_gemm with bf16 products: A and B rounded to bf16 (round to
 * nearest even) before v_mfma_f32_16x16x32_bf16, fp32 accumulation and
 * epilogue (the reference's USE_BF16 build, pufferlib.cu precision_t = bf16
 * with cuBLAS fp32 compute).  Shapes that break the 128-bit operand rules
 * run the fp32 kernel.                                                     */
int ptcg_kernel_gemm_bf16(int M, int N, int K, const float* A, int64_t lda, int a_t,
                          const float* B, int64_t ldb, int b_t, float* C, int64_t ldc, int epi,
                          const float* bias, const float* R, int64_t ldr, float* C2, int64_t ldc2,
                          float* workspace, int64_t workspace_floats, void* stream);

/* weight gradient of a linear layer Y = X W^T + b (pt_linear_bwd's dW / db,
 * ptcg_kernels.cuh:81-108): dW (out, in) = dY^T X, db (out) = column sums of
 * dY (optional, NULL to skip), both overwritten and summed in a fixed order.
 * dY (rows, out) at row stride lddy, X (rows, in) at row stride ldx.
 * workspace: split-K partials, up to 512 tiles of out*in + out floats.      */
int ptcg_kernel_gemm_dw(int rows, int in, int out, const float* dY, int64_t lddy,
                        const float* X, int64_t ldx, float* dW, float* db,
                        float* workspace, int64_t workspace_floats, void* stream);

/* ptcg_kernel_gemm_dw over a device row count, as the sync-free model's
 * weight gradients run: rows is the host's bound, *rows_dev (device int,
 * <= rows) the rows summed.  The launch is sized for the bound's K splits;
 * the split count actually used is the same rule applied to the device
 * count (at most the launched count).
 * No reference counterpart: the sync-free layout's own launch form.        */
int ptcg_kernel_gemm_dw_rows_dev(int rows, int in, int out, const float* dY, int64_t lddy,
                                 const float* X, int64_t ldx, float* dW, float* db, const int* rows_dev,
                                 float* workspace, int64_t workspace_floats, void* stream);

/* ptcg_kernel_gemm_dw with bf16 products (dY and X rounded to bf16 before
 * the MFMA, fp32 accumulation); db sums the unrounded fp32 dY.            */
int ptcg_kernel_gemm_dw_bf16(int rows, int in, int out, const float* dY, int64_t lddy,
                             const float* X, int64_t ldx, float* dW, float* db,
                             float* workspace, int64_t workspace_floats, void* stream);

/* Products on operands STORED in bf16 (the mixed-precision variant's
 * activations, pufferlib.cu precision_t = bf16; uint16 bit patterns),
 * v_mfma_f32_16x16x32_bf16 with fp32 accumulation.
 * ptcg_kernel_gemm_bs: C (M, N) = epi(A B^T), A (M, K) at row stride lda,
 * B (N, K) at row stride ldb, K, lda, ldb multiples of 8, A and B 16 B
 * aligned; epilogues STORE (fp32 or bf16 C), BIAS (bf16 C), BIAS_RESID
 * (fp32 C and R), BIAS_GELU_D (bf16 C = gelu'(z), C2 = gelu(z)), MUL (bf16 C
 * and R); out_bf16 selects the output type; bias fp32.
 * ptcg_kernel_gemm_dw_bs: dW (out, in) = dY^T X and db = column sums of dY
 * (optional), fp32, dY (rows, out) and X (rows, in) bf16; out, in, lddy,
 * ldx multiples of 8; workspace as ptcg_kernel_gemm_dw.                    */
int ptcg_kernel_gemm_bs(int M, int N, int K, const void* A, int64_t lda, const void* B, int64_t ldb,
                        void* C, int64_t ldc, int epi, int out_bf16, const float* bias, const void* R,
                        int64_t ldr, void* C2, int64_t ldc2, void* stream);
int ptcg_kernel_gemm_dw_bs(int rows, int in, int out, const void* dY, int64_t lddy, const void* X,
                           int64_t ldx, float* dW, float* db, float* workspace, int64_t workspace_floats,
                           void* stream);

/* deterministic column sums out[n] = sum_m X[m*ldx+n] (pt_bias_grad,
 * ptcg_kernels.cuh:87-96); workspace >= ceil(M/256)*N floats.              */
int ptcg_kernel_colsum(const float* X, int64_t ldx, int M, int N, float* out,
                       float* workspace, int64_t workspace_floats, void* stream);

/* LayerNorm, eps 1e-5 (pt_ln_fwd / pt_ln_bwd, ptcg_kernels.cuh:132-218).
 * bwd: dx = LN'(dy) [+ dres]; dw, db overwritten; workspace >=
 * 2048*D floats.                                                          */
int ptcg_kernel_layernorm_fwd(const float* x, const float* w, const float* b, float* y,
                              float* mean, float* rstd, int rows, int D, void* stream);
/* A pre-LN block's residual product fused with the LayerNorm that reads its
 * output: C (rows, 256) = A (rows, K) W^T + bias + R, then y = LN(C) lnw +
 * lnb with mean / rstd (eps 1e-5), in one launch.  W (256, K) and A at row
 * stride K; R, C, y at row stride 256; K a multiple of 16; 16 B aligned.
 * bf16 = 1: A, W and y hold bf16 (bf16 products, fp32 accumulation, C, R,
 * statistics fp32; K a multiple of 32).  rows_dev (nullable): a device row
 * count, rows < it are processed.
 * Replaces the residual add + LayerNorm pair of the block forward
 * (ptcg_model.cu's pt_linear with residual then pt_ln_fwd,
 * ptcg_kernels.cuh:42-108,132-175).                                       */
int ptcg_kernel_gemm_resid_ln(int rows, int K, const void* A, const void* W, const float* bias,
                              const float* R, float* C, const float* lnw, const float* lnb, void* y,
                              float* mean, float* rstd, int bf16, const int* rows_dev, void* stream);
int ptcg_kernel_layernorm_bwd(const float* dy, const float* x, const float* w,
                              const float* mean, const float* rstd, const float* dres,
                              float* dx, float* dw, float* db, int rows, int D,
                              float* workspace, int64_t workspace_floats, void* stream);
/* A bf16 block's dX product fused with the LayerNorm backward that reads
 * it: dy (rows, 256) = dY (rows, K) WT^T with dY and the weight copy WT
 * (256, K) bf16 at row stride K (K a multiple of 32, 16 B aligned), then
 * dx = LN'(dy) [+ dres] at row stride 256, its bf16 copy dxh (nullable),
 * dw / db overwritten; workspace >= 2048*ceil(rows/64) floats.  rows_dev
 * (nullable): a device row count, rows < it are processed (dw / db over
 * those rows only).  Replaces the QKV / FFN1 dX product and the LayerNorm
 * backward after it (ptcg_model.cu's dX pt_linear then pt_ln_bwd,
 * ptcg_kernels.cuh:176-218).                                              */
int ptcg_kernel_gemm_dx_layernorm_bwd(int rows, int K, const void* dY, const void* WT, const float* x,
                                      const float* w, const float* mean, const float* rstd,
                                      const float* dres, float* dx, void* dxh, float* dw, float* db,
                                      float* workspace, int64_t workspace_floats, const int* rows_dev,
                                      void* stream);

/* Masked MHSA over (N, L, 3D) qkv rows, keep (N, L) key mask (1 keep / 0
 * masked), fused per (sample, head) (ptcg_model3.cu:18-30, 63-91).
 * fwd: ctx (N, L, D), lse (N, H, L).  bwd: dqkv (N, L, 3D) from dctx.     */
int ptcg_kernel_attention_fwd(const float* qkv, const float* keep, float* ctx, float* lse,
                              int N, int L, int H, int Dh, void* stream);
int ptcg_kernel_attention_bwd(const float* qkv, const float* keep, const float* ctx,
                              const float* lse, const float* dctx, float* dqkv,
                              int N, int L, int H, int Dh, void* stream);
/* the same with bf16 products (the reference's USE_BF16 attention, whose
 * batched products run on precision_t = bf16): S, P.V and the backward's
 * products on v_mfma_f32_16x16x16_bf16 with operands rounded to bf16 (RNE),
 * softmax, log-sum-exp and accumulation in fp32.                          */
int ptcg_kernel_attention_fwd_bf16(const float* qkv, const float* keep, float* ctx, float* lse,
                                   int N, int L, int H, int Dh, void* stream);
int ptcg_kernel_attention_bwd_bf16(const float* qkv, const float* keep, const float* ctx,
                                   const float* lse, const float* dctx, float* dqkv,
                                   int N, int L, int H, int Dh, void* stream);

/* the backward with its L x L dS tiles in a global scratch instead of LDS
 * (Lp <= 128): LDS holds only Q and dO, so two workgroups share a CU.  The
 * scratch takes ptcg_kernel_attention_bwd_ws_bytes(N, L, H, Dh, bf16) bytes
 * (0: the shape takes the recompute pair, which needs none); bf16 selects
 * the bf16-product kernels of ptcg_kernel_attention_bwd_bf16.  The model's
 * training backward runs this form.                                      */
int64_t ptcg_kernel_attention_bwd_ws_bytes(int N, int L, int H, int Dh, int bf16);
int ptcg_kernel_attention_bwd_ws(const float* qkv, const float* keep, const float* ctx,
                                 const float* lse, const float* dctx, float* dqkv,
                                 int N, int L, int H, int Dh, int bf16, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/* which attention kernels a row length takes: bit 0 forward (MFMA), bit 1
 * backward with the L x L dS tile parked in LDS (Lp <= 128), bit 2 backward
 * recomputing S and dP per query stripe (longer rows); -1 unsupported.     */
int ptcg_kernel_attention_path(int L, int Dh);

/* Launch timing: between begin and end, every GEMM, LayerNorm and Adam
 * launch (up to max_launches in all) is bracketed by a HIP event pair on its
 * own stream.  end waits for the events and returns the GEMM launches'
 * summed kernel time (ms), their number and their summed 2*M*N*K.
 * No reference counterpart (measurement only).                             */
int ptcg_profile_begin(int max_launches);
int ptcg_profile_end(double* total_ms, int* launches, double* flops);

/* Totals of one launch class of the last closed profile: summed kernel time
 * (ms), launches, and summed algorithmic amount -- flops for class 0, HBM
 * bytes for the others:
 *   0 GEMM; 1 LayerNorm forward (8d+8 B per row + weights);
 *   2 LayerNorm backward (12d+8 B per row, +4d with a residual gradient);
 *   3 Adam norm pass (4 B per parameter); 4 Adam update (28 B per parameter);
 *   5 whole Muon step (Newton-Schulz flops); 6 Muon's Newton-Schulz GEMM
 *   launches (flops; not counted in class 0); 7 token-concat gather (the
 *   rows written and the obs floats read); 8 PPO loss with its masked
 *   softmax (the (A+1) outputs, A mask floats and per-row inputs read, the
 *   (A+1) gradient and ratio / new value written).                        */
int ptcg_profile_class(int cls, double* total_ms, int* launches, double* amount);

#ifdef __cplusplus
}
#endif
#endif /* PTCG_AMD_KERNELS_H */
