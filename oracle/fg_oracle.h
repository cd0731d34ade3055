/*
 * fg_oracle.h -- CPU restatement of ferrograd's fused-training-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the timed
 * CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library (ferrograd_amd) never
 * links or calls it.
 *
 * The reference (bobbothe2nd/ferrograd) is Rust that generates GPU source at
 * run time; it has no CPU implementation and cannot be built in this image
 * (no cargo/rustc, crates.io dependencies absent).  Every function below
 * restates the semantics of the reference file:line it cites, with the
 * reference's documented defects corrected (see each comment).
 *
 * Conventions: row-major fp32, last dimension contiguous, leading dimension
 * given in elements.  All functions are pure CPU code (OpenMP across rows).
 */
#ifndef FG_ORACLE_H
#define FG_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GEMM operand layouts.
 *   NN: C = A.B    A[M][K] lda, B[K][N] ldb   (forward;  matmul/generic.rs:98-149)
 *   NT: C = A.B^T  A[M][K] lda, B[N][K] ldb   (dA = dC.B^T; matmul/mod.rs:75-84)
 *   TN: C = A^T.B  A[K][M] lda, B[K][N] ldb   (dB = A^T.dC; matmul/mod.rs:85-94) */
enum { FGO_NN = 0, FGO_NT = 1, FGO_TN = 2 };
enum { FGO_ACT_NONE = 0, FGO_ACT_RELU = 1, FGO_ACT_GELU = 2 };

/* C[M][N] = op(A).op(B), fp32 products accumulated in fp32 with fused
 * multiply-add in ascending k, as the reference's K loop does
 * (generic.rs:251-314, fmaf contraction from kernel/optimize.rs:31-87). */
void fgo_gemm(int layout, int M, int N, int K, const float *A, int lda,
              const float *B, int ldb, float *C, int ldc);

/* Z = C + bias (row broadcast; bias may be NULL), H = act(Z).
 * Z or H may alias C.  Bias broadcast is new (reference binary.rs:53-63 has
 * none); activation formulas from unary.rs:436-490 (ReLU) and
 * unary.rs:492-587 (GELU tanh form, constants 0.7978846 and 0.044715). */
void fgo_bias_act(int M, int N, const float *C, int ldc, const float *bias,
                  int act, float *Z, float *H);

/* Scalar activation and its derivative w.r.t. the pre-activation z.
 * ReLU' = [z > 0] (reference unary.rs:460-469 tests its own output >= 0,
 * which is always true -- corrected).  GELU' is the exact derivative of the
 * tanh form in terms of z (reference unary.rs:588-714 substitutes tanh(u) for
 * x -- corrected). */
float fgo_act(int act, float z);
float fgo_act_grad(int act, float z);

/* dZ[i] = dH[i] * act'(Z[i]) over n elements. */
void fgo_act_bwd(int act, int64_t n, const float *dH, const float *Z, float *dZ);

/* dbias[j] = sum_i dZ[i][j]  (new; reference has no broadcast). Accumulated
 * in double, rounded once. */
void fgo_bias_grad(int M, int N, const float *dZ, int ld, float *dbias);

/* Row softmax + cross-entropy, forward and backward, one pass per row.
 *   m_r = max_c x, s_r = sum_c exp(x - m_r), lse_r = m_r + log(s_r)
 *   row_loss[r] = lse_r - x[r][label_r]           (= -log p_label, stable)
 *   dlogits[r][c] = grad_scale * (exp(x - m_r)/s_r - [c == label_r])
 *   argmax[r] = first c with x[r][c] == m_r
 * Follows softmax.rs:112-446 (max-subtracted exponentials) and
 * basic_loss.rs:91-133 (u32 label per row; grad p - onehot), with the CE
 * gradient emitted directly instead of being pushed through the softmax
 * Jacobian a second time (defect in basic_loss.rs + softmax.rs:448-688).
 * Any of row_loss / dlogits / argmax may be NULL.  Returns the mean loss
 * (double). */
double fgo_softmax_ce(int R, int C, const float *x, int ldx, const uint32_t *labels,
                      float grad_scale, float *row_loss, float *dlogits,
                      int ldd, uint32_t *argmax);

/* Plain row softmax y = exp(x - max) / sum (softmax.rs:112-446). */
void fgo_softmax(int R, int C, const float *x, float *y);
/* Softmax backward dx = y * (dy - sum_c dy*y) over every column
 * (softmax.rs:448-688, whose second loop restarts at column 0 -- corrected). */
void fgo_softmax_bwd(int R, int C, const float *y, const float *dy, float *dx);

/* SGD (basic_optim.rs:3-31, lr read from meta[0] in kernel/optim.rs:119-131):
 *   w = w - fl(g * lr);  g = 0 when zero_grad. */
void fgo_sgd(int64_t n, float *w, float *g, float lr, int zero_grad);

/* Adam (absent in the reference; PyTorch torch.optim.Adam without weight
 * decay, eps outside the square root).  Per element, in this fp32 order:
 *   m = b1*m + (1-b1)*g
 *   v = b2*v + (1-b2)*(g*g)
 *   p = p - step_size * m / (sqrt(v) * inv_sqrt_bc2 + eps)
 * where step_size = lr / (1 - b1^t) and inv_sqrt_bc2 = 1/sqrt(1 - b2^t) are
 * computed in double by fgo_adam_scalars and rounded to fp32 once. */
void fgo_adam_scalars(double lr, double b1, double b2, int step,
                      float *step_size, float *inv_sqrt_bc2);
void fgo_adam(int64_t n, float *p, const float *g, float *m, float *v,
              float b1, float b2, float eps, float step_size,
              float inv_sqrt_bc2);

/* ------------------------------------------------ 16-bit storage types */
/* SimpleDType F16 / BF16 (crates/fused_gpu/src/dispatch/backend/mod.rs:
 * 335-427; conversions by the `half` crate, version 2, at the reference's
 * upload / download boundary: dispatch/mod.rs:614-645).  Restated from the
 * IEEE 754 binary16 definition and the bfloat16 layout (upper 16 bits of a
 * binary32): round to nearest, ties to even; overflow to infinity; NaN stays
 * NaN (quiet). */
enum { FGO_F32 = 0, FGO_F16 = 1, FGO_BF16 = 2 };
uint16_t fgo_f32_to_f16(float x);
float fgo_f16_to_f32(uint16_t h);
uint16_t fgo_f32_to_bf16(float x);
float fgo_bf16_to_f32(uint16_t h);
/* Element-wise conversions of n values (dtype FGO_F16 or FGO_BF16). */
void fgo_to_f32(int dtype, int64_t n, const uint16_t *src, float *dst);
void fgo_from_f32(int dtype, int64_t n, const float *src, uint16_t *dst);

/* 16-bit GEMM with fp32 accumulation (fgo_gemm on the widened operands);
 * then each node value is rounded to the storage type, in the order the
 * reference's nodes produce them: the matmul, the bias add (bias may be
 * NULL), the activation; with accumulate, C = round(C + value).  Z (may be
 * NULL) receives the rounded pre-activation.  The reference's own 16-bit
 * matmul keeps a 16-bit running sum (op/matmul/mod.rs:150-161) -- replaced
 * by the fp32 sum. */
void fgo_gemm_x16(int dtype, int layout, int M, int N, int K,
                  const uint16_t *A, int lda, const uint16_t *B, int ldb,
                  const uint16_t *bias, int act, uint16_t *C, int ldc,
                  uint16_t *Z, int ldz, int accumulate);
/* Backward form: C (=|+=) round(round(sum) * act'(Zs)); the ReLU mask is a
 * select (+0 where Zs <= 0). */
void fgo_gemm_bwd_x16(int dtype, int layout, int M, int N, int K,
                      const uint16_t *A, int lda, const uint16_t *B, int ldb,
                      int act, const uint16_t *Zs, int ldzs, uint16_t *C,
                      int ldc, int accumulate);

/* Number of OpenMP threads the oracle uses. */
int fgo_num_threads(void);
void fgo_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
