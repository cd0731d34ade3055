/*
 * ferrograd_hip.h -- C ABI of the MI355X (gfx950) backend for ferrograd's
 * fused training path.
 *
 * The reference's seam for this path is the Rust trait `GpuBackend`
 * (crates/fused_gpu/src/dispatch/mod.rs:161-261) implemented by
 * `rocm::GpuContext` (crates/fused_gpu/src/dispatch/backend/rocm/mod.rs:81-429)
 * plus the graph/plug-in types of crates/fused_gpu/src/dispatch/backend/mod.rs.
 * Each entry point below names the reference interface it replaces.
 *
 * Conventions
 *  - Every function returns an fg_status (0 = success).  On failure the
 *    message is available from fg_last_error_msg() on the same thread.
 *  - Sizes are in bytes unless named otherwise; tensors are row-major fp32
 *    with the last dimension contiguous; leading dimensions are in elements.
 *  - Pointers named `d_*` or typed as device tensors are device addresses;
 *    all device work is enqueued on the context's stream, asynchronously,
 *    in call order.  fg_sync() waits for it.
 *  - No call allocates device memory except the fg_buf_*, fg_mt_create,
 *    fg_ctx_reserve_workspace and fg_plan_create entry points, the first
 *    fg_plan_optim / fg_plan_capture_step after inputs are (re)bound (they
 *    build the optimiser's tensor list), and the first call of a direct
 *    kernel that needs more workspace than the context holds.
 */
#ifndef FERROGRAD_HIP_H
#define FERROGRAD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: a subset of fused_gpu::errors::ErrorKind
 * (crates/fused_gpu/src/errors.rs:102-140), one code per kind this backend
 * can raise. */
typedef enum fg_status {
    FG_OK = 0,
    FG_ERR_INVALID_ARGUMENT = 1, /* ErrorKind::InvalidArgument           */
    FG_ERR_OUT_OF_MEMORY = 2,    /* ErrorKind::OutOfMemory               */
    FG_ERR_UNSUPPORTED = 3,      /* ErrorKind::UnsupportedFeature        */
    FG_ERR_DEVICE = 4,           /* ErrorKind::DeviceError (HIP status)  */
    FG_ERR_SHAPE = 5,            /* ErrorKind::ShapeMismatch             */
    FG_ERR_GRAPH = 6,            /* ErrorKind::ComputeGraphError         */
    FG_ERR_INTERNAL = 7,         /* ErrorKind::InternalError             */
    FG_ERR_NO_DEVICE = 8,        /* ErrorKind::NoDevice                  */
    FG_ERR_OUT_OF_BOUNDS = 9,    /* ErrorKind::OutOfBounds               */
    FG_ERR_SERIALIZATION = 10,   /* ErrorKind::SerializationError        */
    FG_ERR_FILE_NOT_FOUND = 11   /* ErrorKind::FileNotFound              */
} fg_status;

/* Message of the last failing call on this thread ("" if none).  Replaces
 * the `msg`/`ctx` fields of fused_gpu::errors::Error (errors.rs:13-19). */
const char *fg_last_error_msg(void);
/* Library ABI version (major*10000 + minor*100 + patch). */
int fg_version(void);

/* ------------------------------------------------------------- context */
typedef struct fg_ctx fg_ctx;

/* Target flags reported by fg_ctx_target (TargetFlags, dispatch/mod.rs:32-60). */
#define FG_TARGET_LIN_ACC 0x1u /* matrix cores present (MFMA)           */

/* Open `device` and bind a stream.  `stream` is an existing hipStream_t to
 * enqueue on, or NULL to create a private default-priority stream.
 * Replaces rocm::GpuContext::new (rocm/mod.rs:57-79). */
int fg_ctx_create(int device, void *stream, fg_ctx **out);
int fg_ctx_destroy(fg_ctx *ctx);
/* Architecture name (e.g. "gfx950"), FG_TARGET_* flags and CU count.
 * Replaces GpuBackend::target_spec (dispatch/mod.rs:161-170). */
int fg_ctx_target(fg_ctx *ctx, char *arch, size_t arch_len, uint32_t *flags,
                  int *cu_count);
/* The hipStream_t work is enqueued on. */
int fg_ctx_stream(fg_ctx *ctx, void **stream);
/* Pre-size the context's scratch workspace so later direct-kernel calls
 * (and graph capture) never allocate.  A GEMM of few output tiles and a long
 * K splits K into this workspace when it already holds the slices (fp32 or
 * fp32 sums of a 16-bit GEMM, M x N floats per slice); it is never grown for
 * that, so a larger workspace can change which GEMMs split. */
int fg_ctx_reserve_workspace(fg_ctx *ctx, uint64_t bytes);
/* GpuBackend::sync / is_ready (rocm/mod.rs:398-400). */
int fg_sync(fg_ctx *ctx);
int fg_is_ready(fg_ctx *ctx, int *ready);

/* ------------------------------------------------------------- buffers */
typedef struct fg_buf fg_buf;

/* GpuBackend::alloc / alloc_zeroed / alloc_init (dispatch/mod.rs:161-200).
 * Sizes are u64 bytes (the reference's are u32). */
int fg_buf_alloc(fg_ctx *ctx, uint64_t bytes, fg_buf **out);
int fg_buf_alloc_zeroed(fg_ctx *ctx, uint64_t bytes, fg_buf **out);
int fg_buf_alloc_init(fg_ctx *ctx, const void *src, uint64_t bytes, fg_buf **out);
int fg_buf_free(fg_buf *buf);
/* Buffer::size_bytes (tensor.rs:125-198). */
uint64_t fg_buf_size_bytes(const fg_buf *buf);
/* Device address of the buffer's first byte. */
void *fg_buf_device_ptr(const fg_buf *buf);
/* GpuBackend::upload / download / copy (rocm/mod.rs:184-205, 402-421):
 * synchronous with respect to the host buffer. */
int fg_upload(fg_ctx *ctx, fg_buf *dst, const void *src, uint64_t bytes,
              uint64_t dst_off);
int fg_download(fg_ctx *ctx, const fg_buf *src, void *dst, uint64_t bytes,
                uint64_t src_off);
int fg_copy(fg_ctx *ctx, const fg_buf *src, fg_buf *dst);
/* Fill `count` u32 words of a buffer with `value` (a small fill kernel,
 * safe under stream capture). */
int fg_fill_u32(fg_ctx *ctx, void *d_dst, uint32_t value, uint64_t count);

/* ------------------------------------------------- direct kernel calls */
/* Operand layouts of the matmul lowering (ferrograd-nn op/matmul/mod.rs:17-188):
 *   NN: C = A.B     A[M][K], B[K][N]   forward          (generic.rs:98-149)
 *   NT: C = A.B^T   A[M][K], B[N][K]   dA = dC.B^T      (mod.rs:75-84)
 *   TN: C = A^T.B   A[K][M], B[K][N]   dB = A^T.dC      (mod.rs:85-94)   */
typedef enum fg_layout { FG_NN = 0, FG_NT = 1, FG_TN = 2 } fg_layout;
/* Activations fused in GEMM epilogues (relu: unary.rs:436-490,
 * gelu tanh form: unary.rs:492-733). */
typedef enum fg_act { FG_ACT_NONE = 0, FG_ACT_RELU = 1, FG_ACT_GELU = 2 } fg_act;

/* Forward GEMM with fused epilogue:
 *   Zv = op(A).op(B) (+ bias[col] if d_bias) ;  C = act(Zv)
 *   if d_Z: Z = Zv (pre-activation saved for backward)
 *   if accumulate: C += act(Zv) instead of C = act(Zv) (requires act NONE)
 * An output of few tiles with a long K (and the backward form below) may be
 * split over K into the context's workspace when what is already reserved
 * holds the slices (it is never grown for this), then summed in a fixed
 * order: deterministic, within the GEMM tolerance of the unsplit sum.
 * Replaces the matmul-rooted fused kernel (forward.rs:298-464 with
 * generic.rs:13-325) plus the bias/activation consumers inlined after it. */
int fg_gemm_f32(fg_ctx *ctx, int layout, int M, int N, int K,
                const float *d_A, int lda, const float *d_B, int ldb,
                const float *d_bias, int act, float *d_C, int ldc,
                float *d_Z, int ldz, int accumulate);

/* Backward GEMM with the activation derivative fused in the epilogue:
 *   C = (op(A).op(B)) * act'(Zs)        (elementwise, Zs[M][N] ld ldzs)
 * or C += ... when accumulate.  With act NONE, Zs is ignored.  Used for
 * dZ_prev = (dZ . W^T) * act'(Z_prev): matmul dA (mod.rs:75-84) with the
 * upstream activation's backward (unary.rs) inlined. */
int fg_gemm_bwd_f32(fg_ctx *ctx, int layout, int M, int N, int K,
                    const float *d_A, int lda, const float *d_B, int ldb,
                    int act, const float *d_Zs, int ldzs, float *d_C, int ldc,
                    int accumulate);

/* Backward of a Linear layer through its activation, C = act(X.W + bias):
 *   dZ = dC * act'(Zs)
 *   dX (=|+=) dZ . W^T        [M][K], ld lddx   (NULL: skipped)
 *   dW (=|+=) X^T . dZ        [K][N], ld lddw   (NULL: skipped)
 *   dbias (=|+=) colsum(dZ)   [N]               (NULL: skipped)
 * X[M][K] ld ldx, W[K][N] ld ldw, Zs and dC [M][N] (ld ldzs, lddc).  act is
 * FG_ACT_RELU, FG_ACT_GELU or FG_ACT_NONE (Zs unused, dZ = dC).  For ReLU, Zs
 * may be the forward output C itself: [C > 0] == [Z > 0].  `accumulate`
 * applies to dX, dW and dbias.  Two ways to apply act':
 *   d_dZ given ([M][N], ld lddz): one HBM pass writes dZ there and sums its
 *     columns into dbias, then plain GEMMs read dZ (the faster way for large
 *     layers: one extra pass of 12 bytes per element);
 *   d_dZ NULL: dZ is never stored -- each dC tile is multiplied by act'(Zs)
 *     as the two GEMMs load it, and dbias is summed from the dW GEMM's
 *     scaled tiles (no extra memory; the GEMMs run some per cent slower).
 * Replaces the matmul backward (op/matmul/mod.rs:75-125 driven by
 * kernel/backward.rs:229-371), which evaluates dC inline on every tile load,
 * with the activation's backward inlined there (relu unary.rs:456-469, with
 * the mask corrected to [z > 0]; gelu unary.rs:588-714, corrected to the
 * derivative in z). */
int fg_linear_bwd_f32(fg_ctx *ctx, int act, int M, int N, int K,
                      const float *d_X, int ldx, const float *d_W, int ldw,
                      const float *d_Zs, int ldzs, const float *d_dC, int lddc,
                      float *d_dX, int lddx, float *d_dW, int lddw, float *d_dbias,
                      int accumulate, float *d_dZ, int lddz);

/* A matmul node's two gradients from its upstream gradient dZ[M][N] (the
 * product C = X.W with X[M][K], W[K][N]), all outputs (=|+=) by accumulate:
 *   dW = X^T.dZ [K][N] ld lddw, and dbias = colsum(dZ) unless d_dbias is NULL;
 *   dX = (dZ.W^T) * act'(Zs) [M][K] ld lddx, Zs[M][K] the pre-activation of
 *   X's producer (act NONE: the plain product, Zs ignored).
 * Both GEMMs read dZ and write different tensors, so when the kernels they
 * would take alone pair (the large layers' 8-wave tiles, the 128x64 tiles,
 * the small tiles), one launch runs both, each part exactly as its own call:
 * fg_gemm_dw_f32 + fg_gemm_bwd_f32 give the same bits.  Otherwise the two
 * calls run in turn.  Replaces the two matmul backward kernels
 * (op/matmul/mod.rs:75-94, Some(0) and Some(1)) that
 * kernel/backward.rs:229-371 generates for one matmul node, with the
 * producer activation's backward (unary.rs) inlined into dA. */
int fg_matmul_bwd_f32(fg_ctx *ctx, int M, int N, int K,
                      const float *d_X, int ldx, const float *d_W, int ldw,
                      const float *d_dZ, int lddz, int act, const float *d_Zs, int ldzs,
                      float *d_dX, int lddx, float *d_dW, int lddw, float *d_dbias,
                      int accumulate);

/* Element types of tensors: SimpleDType F32 / F16 / BF16
 * (crates/fused_gpu/src/dispatch/backend/mod.rs:335-427). 16-bit tensors are
 * stored as 16-bit words; kernels compute in fp32 and round to the storage
 * type (nearest even) wherever a node value is stored. */
typedef enum fg_dtype { FG_DTYPE_F32 = 0, FG_DTYPE_F16 = 1, FG_DTYPE_BF16 = 2 } fg_dtype;

/* 16-bit GEMMs (dtype FG_DTYPE_F16 or FG_DTYPE_BF16 for every operand and
 * output): the same contract as fg_gemm_f32 / fg_gemm_bwd_f32, with the
 * products summed in fp32 on the MFMA units and each node value -- the
 * matmul, the bias add, the activation, C += -- rounded to the storage
 * type.  Replaces the 16-bit instances of the matmul lowering
 * (op/matmul/mod.rs:150-161, generic.rs:13-325), whose running sum is
 * itself 16-bit. Leading dimensions are in elements. */
int fg_gemm_x16(fg_ctx *ctx, int dtype, int layout, int M, int N, int K,
                const void *d_A, int lda, const void *d_B, int ldb,
                const void *d_bias, int act, void *d_C, int ldc,
                void *d_Z, int ldz, int accumulate);
int fg_gemm_bwd_x16(fg_ctx *ctx, int dtype, int layout, int M, int N, int K,
                    const void *d_A, int lda, const void *d_B, int ldb,
                    int act, const void *d_Zs, int ldzs, void *d_C, int ldc,
                    int accumulate);

/* The weight and bias gradients of a Linear layer in one launch:
 *   C (=|+=) A^T.B        A[K][M] lda, B[K][N] ldb (the TN layout: dW = X^T.dZ)
 *   colsum[n] (=|+=) sum_k B[k][n]   (dbias = column sums of dZ; may be NULL)
 * The column sums come from the B tiles the GEMM already stages, so dbias
 * costs no extra pass over dZ (the reference has no bias broadcast, see
 * binary.rs:53-63; its dB is matmul/mod.rs:85-94). */
int fg_gemm_dw_f32(fg_ctx *ctx, int M, int N, int K, const float *d_A, int lda,
                   const float *d_B, int ldb, float *d_C, int ldc, int accumulate,
                   float *d_colsum, int colsum_accumulate);

/* The same for 16-bit tensors (dtype FG_DTYPE_F16 / FG_DTYPE_BF16 for every
 * operand, colsum included): C as fg_gemm_x16 in the TN layout; colsum[n]
 * (=|+=) sum_k B[k][n] summed in fp32 and rounded to dtype once (with
 * colsum_accumulate: round(colsum + sum)). Shapes off the pipelined
 * path (K not a multiple of the tile depth, unaligned rows) take the GEMM
 * plus fg_bias_grad's reduction: the same values up to the order of the
 * fp32 sums. Replaces the 16-bit dB lowering (matmul/mod.rs:85-94) and the
 * bias add's backward, which the reference lacks (binary.rs:53-63). */
int fg_gemm_dw_x16(fg_ctx *ctx, int dtype, int M, int N, int K, const void *d_A, int lda,
                   const void *d_B, int ldb, void *d_C, int ldc, int accumulate,
                   void *d_colsum, int colsum_accumulate);

/* fg_matmul_bwd_f32 for 16-bit tensors (dtype FG_DTYPE_F16 / FG_DTYPE_BF16
 * for every operand and output; leading dimensions in elements): dW and
 * dbias as fg_gemm_dw_x16, dX as fg_gemm_bwd_x16 in the NT layout, one
 * launch when both take the large layers' pipelined kernels unsplit (the
 * same bits as the two calls), else the two calls in turn.  Replaces the
 * 16-bit instances of the matmul backward (op/matmul/mod.rs:75-94). */
int fg_matmul_bwd_x16(fg_ctx *ctx, int dtype, int M, int N, int K,
                      const void *d_X, int ldx, const void *d_W, int ldw,
                      const void *d_dZ, int lddz, int act, const void *d_Zs, int ldzs,
                      void *d_dX, int lddx, void *d_dW, int lddw, void *d_dbias,
                      int accumulate);

/* dbias[j] (=|+=) sum_i dZ[i][j]: the bias-add's backward (new broadcast
 * op; reference binary.rs:53-63 has none). Deterministic order. */
int fg_bias_grad_f32(fg_ctx *ctx, int M, int N, const float *d_dZ, int ld,
                     float *d_dbias, int accumulate);

/* Same reduction over dZ of element type dtype (fp32 sums, the result
 * rounded to dtype once). */
int fg_bias_grad(fg_ctx *ctx, int dtype, int M, int N, const void *d_dZ, int ld,
                 void *d_dbias, int accumulate);

/* fg_bias_grad without any device allocation: no counterpart in the
 * reference.  For callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The same
 * launches and bits as fg_bias_grad; its partial sums go to a fixed 4 MiB
 * device array of the library (one per GPU, held until the process ends)
 * instead of the context workspace, so N is limited to 1,048,576 columns
 * (FG_ERR_OUT_OF_BOUNDS beyond).  Calls on one GPU share that array: calls
 * that overlap on one GPU (other streams or threads) race and must be
 * ordered by the caller. */
int fg_bias_grad_noalloc(fg_ctx *ctx, int dtype, int M, int N, const void *d_dZ, int ld,
                         void *d_dbias, int accumulate);

/* dZ[i] = dH[i] * act'(Z[i]) over n elements (unary backward, unary.rs). */
int fg_act_bwd_f32(fg_ctx *ctx, int act, uint64_t n, const float *d_dH,
                   const float *d_Z, float *d_dZ);

/* Fused row softmax + cross-entropy, forward and backward, one HBM read of
 * the logits (softmax.rs:112-446 + basic_loss.rs:91-133 + loss.rs:12-165):
 *   row_loss[r] = logsumexp(x_r) - x_r[label_r]
 *   mean_loss[0] = mean_r row_loss[r]
 *   dlogits[r][c] = grad_scale * (softmax(x_r)[c] - [c == label_r])
 *   argmax[r] = lowest c attaining max_c x_r[c]
 * Any output pointer may be NULL to skip it. labels[r] must be < C. */
int fg_softmax_ce_f32(fg_ctx *ctx, const float *d_logits, int ldx,
                      const uint32_t *d_labels, int R, int C, float grad_scale,
                      float *d_row_loss, float *d_mean_loss, float *d_dlogits,
                      int ldd, uint32_t *d_argmax);

/* Same, with logits and dlogits of element type dtype (FG_DTYPE_*): fp32
 * arithmetic, dlogits rounded to dtype once; row_loss / mean_loss stay fp32. */
int fg_softmax_ce(fg_ctx *ctx, int dtype, const void *d_logits, int ldx,
                  const uint32_t *d_labels, int R, int C, float grad_scale,
                  float *d_row_loss, float *d_mean_loss, void *d_dlogits, int ldd,
                  uint32_t *d_argmax);

/* Plain row softmax y = softmax(x) and its backward
 * dx (=|+=) y * (dy - sum(dy*y)) (softmax.rs:112-446, 448-688). */
int fg_softmax_f32(fg_ctx *ctx, const float *d_x, int R, int C, float *d_y);
int fg_softmax_bwd_f32(fg_ctx *ctx, const float *d_y, const float *d_dy, int R,
                       int C, float *d_dx, int accumulate);
/* The same two over tensors of element type dtype (fp32 arithmetic). */
int fg_softmax(fg_ctx *ctx, int dtype, const void *d_x, int R, int C, void *d_y);
int fg_softmax_bwd(fg_ctx *ctx, int dtype, const void *d_y, const void *d_dy, int R,
                   int C, void *d_dx, int accumulate);

/* ----------------------------------------- multi-tensor optimiser lists */
/* One launch updates every tensor of the list.  Replaces the per-tensor
 * optimiser kernels captured one launch per input tensor
 * (kernel/optim.rs:12-158, rocm/mod.rs:268-322), with per-tensor sizes
 * (the reference derives every size from the root node's shape). */
typedef struct fg_mt fg_mt;
/* params/grads: n device pointers each; m/v: n device pointers each for Adam
 * state, or NULL for SGD; sizes: elements per tensor. */
int fg_mt_create(fg_ctx *ctx, int n, float *const *d_params,
                 float *const *d_grads, float *const *d_m, float *const *d_v,
                 const uint64_t *sizes, fg_mt **out);
/* Same, with an element type per tensor (dtypes[i], FG_DTYPE_*; NULL = all
 * fp32) for its parameter and gradient; m / v stay fp32.  A 16-bit
 * parameter is updated in fp32 and rounded to its type once per step. */
int fg_mt_create_x(fg_ctx *ctx, int n, const int *dtypes, void *const *d_params,
                   void *const *d_grads, float *const *d_m, float *const *d_v,
                   const uint64_t *sizes, fg_mt **out);
int fg_mt_destroy(fg_mt *mt);
/* SGD (basic_optim.rs:3-31): w -= fl(g*lr); g = 0 when zero_grad. */
int fg_sgd_step(fg_ctx *ctx, fg_mt *mt, float lr, int zero_grad);
/* Adam (PyTorch formula, bias-corrected; absent in the reference):
 *   m = b1 m + (1-b1) g ; v = b2 v + (1-b2) g^2
 *   p -= (lr/(1-b1^t)) m / (sqrt(v)/sqrt(1-b2^t) + eps)
 * `step` is t >= 1; bias corrections are computed in double on the host. */
int fg_adam_step(fg_ctx *ctx, fg_mt *mt, float lr, float b1, float b2,
                 float eps, int step, int zero_grad);
/* Same update with precomputed fp32 step_size = lr/(1-b1^t) and
 * inv_sqrt_bc2 = 1/sqrt(1-b2^t) (what fg_adam_step derives). */
int fg_adam_step_scalars(fg_ctx *ctx, fg_mt *mt, float b1, float b2, float eps,
                         float step_size, float inv_sqrt_bc2, int zero_grad);

/* Raw host <-> device copies on the context's stream, synchronous with
 * respect to the host buffer (GpuBackend::upload / download for buffers
 * the plan owns, dispatch/mod.rs:161-261). */
int fg_memcpy_h2d(fg_ctx *ctx, void *d_dst, const void *src, uint64_t bytes);
int fg_memcpy_d2h(fg_ctx *ctx, void *dst, const void *d_src, uint64_t bytes);

/* ------------------------------------------------------------ telemetry */
/* Device memory monitor: the gpu_telemetry 0.2 GpuMonitor the reference's
 * example harness uses (crates/ferrograd/examples/matmul_chain3.rs:145-171:
 * start(interval), stop(), samples of heap usage / budget).  A background
 * thread samples hipMemGetInfo on the context's device every interval_us
 * (>= 100): used = total - free, budget = total. */
typedef struct fg_monitor fg_monitor;
int fg_monitor_start(fg_ctx *ctx, int interval_us, fg_monitor **out);
int fg_monitor_stop(fg_monitor *m, int *n_samples);
int fg_monitor_sample(const fg_monitor *m, int index, double *t_s, uint64_t *used,
                      uint64_t *budget);
int fg_monitor_destroy(fg_monitor *m);

/* ------------------------------------------------------- bpat tensor files */
/* fused_gpu::io (crates/fused_gpu/src/io/mod.rs:20-196; layouts in
 * io/headers.rs:1-117): BpatHeader variants in declaration order. */
typedef enum fg_bpat_header {
    FG_BPAT_V0 = 0,      /* "bpat":       u64 rank and dims, f64 data            */
    FG_BPAT_V1 = 1,      /* "BPATv1\0\0": as V0 + CRC-32 per tensor and per file */
    FG_BPAT_V1M = 2,     /* "BPATv1m\0":  u32 rank and dims, f32 data, CRCs      */
    FG_BPAT_V2_F16 = 3,  /* "BPAT\0f16":  u32 rank and dims, f16 data            */
    FG_BPAT_V2_BF16 = 4, /* "BPATbf16":   u32 rank and dims, bf16 data           */
    FG_BPAT_V2_F32 = 5   /* "BPAT\0f32":  u32 rank and dims, f32 data            */
} fg_bpat_header;

/* One device tensor to save: d_ptr holds prod(shape) elements of dtype. */
typedef struct fg_bpat_tensor {
    const void *d_ptr;
    int dtype;          /* FG_DTYPE_* */
    int rank;           /* 0..8 */
    uint32_t shape[8];
} fg_bpat_tensor;

/* save_tensors (io/mod.rs:95-123): writes n <= 255 tensors, converting each
 * to the header's element type (nearest even when narrowing). */
int fg_bpat_save(fg_ctx *ctx, const char *path, int header, int n,
                 const fg_bpat_tensor *tensors);
/* The same from host memory (d_ptr read as a host pointer): for tools and
 * for writing files without a device. */
int fg_bpat_save_host(const char *path, int header, int n, const fg_bpat_tensor *tensors);
/* load_tensors (io/mod.rs:125-160) split in two steps: parse (and verify
 * the CRCs of V1 / V1M) a file into host memory, then upload any of its
 * tensors into caller-owned device memory of a chosen element type. */
typedef struct fg_bpat fg_bpat;
int fg_bpat_open(const char *path, fg_bpat **out);
int fg_bpat_close(fg_bpat *f);
int fg_bpat_info(const fg_bpat *f, int *header, int *count);
/* shape receives up to 8 dims. */
int fg_bpat_tensor_info(const fg_bpat *f, int index, int *rank, uint32_t *shape,
                        uint64_t *numel);
int fg_bpat_read_f32(const fg_bpat *f, int index, float *dst);
int fg_bpat_upload(fg_ctx *ctx, const fg_bpat *f, int index, void *d_dst, int dtype);

/* --------------------------------------------------------------- graph */
/* ----------------------------------------- compiled elementwise kernels */
/* A plan runs each fused elementwise chain (forward, backward, losses) as one
 * launch of an elementwise program: either a kernel generated for the
 * program and compiled at run time with hipRTC -- as the reference compiles
 * every fused kernel it generates (GpuBackend::compile,
 * crates/fused_gpu/src/dispatch/mod.rs:210; rocm/mod.rs:140-170) -- or the
 * library's precompiled interpreter of such programs.  Both give the same
 * bits.  Compiled kernels are kept for the life of the process, one per
 * device and program; a graph capture meeting a program not compiled yet
 * uses the interpreter (fg_plan_capture_step compiles its programs before it
 * captures).  The setting is process-wide; the environment variable
 * FG_ELTWISE_MODE (0, 1 or 2) sets the initial mode, default
 * FG_ELTWISE_COMPILE_LARGE.  No reference counterpart: its backend always
 * compiles. */
#define FG_ELTWISE_INTERPRET 0      /* every program on the interpreter         */
#define FG_ELTWISE_COMPILE_LARGE 1  /* compile programs over >= 2^20 elements   */
#define FG_ELTWISE_COMPILE_ALL 2    /* compile every program                    */
int fg_eltwise_set_mode(int mode, int *previous);
/* Process-wide counts: kernels compiled, launches of compiled kernels,
 * launches of the interpreter (any pointer may be NULL). */
int fg_eltwise_stats(uint64_t *kernels_compiled, uint64_t *compiled_launches,
                     uint64_t *interpreted_launches);

/* Graph IR: the mirror of fused_gpu's Graph / Node / GraphOp
 * (crates/fused_gpu/src/dispatch/backend/mod.rs:499-1316) with the
 * ferrograd-nn builders as a fixed operation enum.  Node ids are creation
 * order (mod.rs:1224-1235); the last node is the forward output. */
typedef struct fg_graph fg_graph;

/* LossType constants (crates/ferrograd-nn/src/loss/basic_loss.rs). */
typedef enum fg_loss {
    FG_LOSS_MSE = 0, /* MEAN_SQUARED_ERROR   (basic_loss.rs:3-27)   */
    FG_LOSS_BCE = 1, /* BINARY_CROSS_ENTROPY (basic_loss.rs:29-89)  */
    FG_LOSS_CE = 2   /* CROSS_ENTROPY        (basic_loss.rs:91-133) */
} fg_loss;

/* OptimType constants: SGD (ferrograd-nn optim/basic_optim.rs:3-31) and
 * Adam (new; absent in the reference). */
typedef enum fg_optim { FG_OPTIM_SGD = 0, FG_OPTIM_ADAM = 1 } fg_optim;

/* Operations of the ferrograd-nn builders (crates/ferrograd-nn/src/op/,
 * re-exported by crates/ferrograd/src/graph.rs:106-159).  BIAS_ADD is new:
 * x[..., N] + b[N] broadcast over rows (the reference's add has no
 * broadcast, binary.rs:53-63); ADD / SUB also accept that broadcast. */
typedef enum fg_op {
    FG_OP_INPUT = 0,
    FG_OP_CONST = 1,
    FG_OP_ADD = 2,
    FG_OP_SUB = 3,
    FG_OP_MUL = 4,
    FG_OP_DIV = 5,
    FG_OP_MATMUL = 6,
    FG_OP_RELU = 7,
    FG_OP_GELU = 8,
    FG_OP_ELU = 9,
    FG_OP_TANH = 10,
    FG_OP_EXP = 11,
    FG_OP_LOG = 12,
    FG_OP_ABS = 13,
    FG_OP_NEG = 14,
    FG_OP_SOFTMAX = 15,
    FG_OP_BIAS_ADD = 16
} fg_op;

/* Input flags (extension): every Input is trainable in ferrograd
 * (kernel/backward.rs:95-106, dispatch/mod.rs:735-744). */
#define FG_INPUT_NO_GRAD 0x1u /* compute no gradient for this input      */
#define FG_INPUT_FROZEN 0x2u  /* compute its gradient, never update it    */

/* Graph::new(loss, optim) (crates/ferrograd/src/graph.rs:34). */
int fg_graph_create(int loss, int optim, fg_graph **out);
int fg_graph_destroy(fg_graph *g);
/* Metadata::new_field (backend/mod.rs:576-620): returns the meta index of a
 * new dimension field (1, 2, ...; index 0 holds the learning rate). */
int fg_graph_new_field(fg_graph *g, uint32_t *field);
/* DefineOps::input(&[fields]) (graph.rs:111): an fp32 input whose dims are
 * meta fields. */
int fg_graph_input(fg_graph *g, const uint32_t *fields, int rank, uint32_t *node);
/* DefineOps::input(&[fields], SimpleDType) (graph.rs:111, backend/mod.rs:
 * 335-427): an input of element type dtype (FG_DTYPE_F32 / F16 / BF16).
 * Operations take the type of their first input. */
int fg_graph_input_x(fg_graph *g, const uint32_t *fields, int rank, int dtype,
                     uint32_t *node);
/* DefineOps::constant_f32 (graph.rs:106-159): a scalar constant. */
int fg_graph_constant_f32(fg_graph *g, float value, uint32_t *node);
/* constant_f16 / constant_bf16 (backend/mod.rs:1293-1310): value rounded to
 * dtype (nearest, ties to even). */
int fg_graph_constant(fg_graph *g, int dtype, float value, uint32_t *node);
/* DefineOps::{add,sub,mul,div,matmul,relu,...,softmax}: node from op and
 * inputs (ids must exist already). */
int fg_graph_op(fg_graph *g, int op, const uint32_t *inputs, int n_inputs, uint32_t *node);
int fg_graph_set_input_flags(fg_graph *g, uint32_t node, uint32_t flags);
int fg_graph_num_nodes(const fg_graph *g, uint32_t *n);
/* Graph::validate (backend/mod.rs:853-975, 1172-1185) against a meta
 * binding [lr_bits, dim1, dim2, ...]; any positive dims are accepted (the
 * reference requires multiples of 16, mod.rs:617-619). */
int fg_graph_validate(const fg_graph *g, const uint32_t *meta, int n_meta);

/* ---------------------------------------------------------------- plan */
/* A lowered, allocated and scheduled graph: replaces Graph::lower +
 * GpuContext::compile + alloc_tensors + schedule (kernel/mod.rs:107-152,
 * dispatch/mod.rs:369-455, 509-575, 664-764).  All plan-owned tensors live
 * in one device arena. */
typedef struct fg_plan fg_plan;

/* Buffer roles (AllocTensors, dispatch/mod.rs:835-845). */
typedef enum fg_role {
    FG_ROLE_FORWARD_OUT = 0,   /* value of the last node                     */
    FG_ROLE_SEED = 1,          /* dL/d(last node)                            */
    FG_ROLE_LOSS = 2,          /* loss_t: per element (MSE/BCE, CE on probs), */
                               /* per row (CE fused with a final softmax)     */
    FG_ROLE_FORWARD_SAVED = 3, /* saved forward values, SaveIndicator order  */
    FG_ROLE_GRAD = 4,          /* grad_tensors, SaveIndicator order          */
    FG_ROLE_INPUT = 5,         /* bound input tensors, input order           */
    FG_ROLE_STATE = 6,         /* optimiser state (Adam m, v per input)      */
    FG_ROLE_MEAN_LOSS = 7,     /* scalar mean loss (CE fused)                */
    FG_ROLE_TARGET = 8         /* bound loss target                          */
} fg_role;

/* ctx may be NULL for a dry plan: lowering only (fg_plan_describe and
 * fg_plan_count work; nothing is allocated and dispatch fails).  A plan
 * keeps ctx: destroy the plan before the context (the Rust binding's
 * Plan<'ctx> lifetime says the same). */
int fg_plan_create(fg_ctx *ctx, const fg_graph *g, const uint32_t *meta, int n_meta,
                   fg_plan **out);
int fg_plan_destroy(fg_plan *p);
int fg_plan_count(const fg_plan *p, int role, int *count);
/* Device address, byte size and node id of a role's index-th tensor. */
int fg_plan_tensor(const fg_plan *p, int role, int index, void **d_ptr, uint64_t *bytes,
                   uint32_t *node);
/* Element type (FG_DTYPE_*) of that tensor: the node's type, except fp32
 * Adam state, fp32 per-row CE losses and u32 labels (reported as F32). */
int fg_plan_tensor_dtype(const fg_plan *p, int role, int index, int *dtype);
/* Bind the index-th input (input order) / the loss target to caller-owned
 * device memory (the reference passes in_tensors and the target to
 * schedule / dispatch_loss, dispatch/mod.rs:664-788).  CE targets are u32
 * labels, one per row of the last node; MSE / BCE targets match its shape. */
int fg_plan_bind_input(fg_plan *p, int index, void *d_ptr, uint64_t bytes);
int fg_plan_bind_target(fg_plan *p, const void *d_ptr, uint64_t bytes);
/* Learning rate (meta field 0, kernel/optim.rs:119-131) and Adam betas/eps. */
int fg_plan_set_lr(fg_plan *p, float lr);
int fg_plan_set_adam(fg_plan *p, float b1, float b2, float eps);
/* dispatch_forward / dispatch_loss / dispatch_backward / dispatch_optim /
 * dispatch_single_optim (dispatch/mod.rs:766-814), enqueued on the stream.
 * After fg_plan_loss with CE on a final softmax, the next fg_plan_backward
 * starts from dlogits = p - onehot (the CE gradient is not pushed through
 * the softmax Jacobian again); otherwise it starts from the seed buffer. */
int fg_plan_forward(fg_plan *p);
int fg_plan_loss(fg_plan *p);
int fg_plan_backward(fg_plan *p);
int fg_plan_optim(fg_plan *p);
int fg_plan_single_optim(fg_plan *p, int input_index);
/* Capture forward + loss + backward + optim into one hipGraph (replayed by
 * fg_plan_launch_step); re-capture after rebinding inputs or target. */
int fg_plan_capture_step(fg_plan *p);
int fg_plan_launch_step(fg_plan *p);
/* Checkpoint of a plan to / from a bpat file (format header as for
 * fg_bpat_save): every Input in input order, then for Adam the m and v of
 * each updated input and a one-element tensor holding the step count.
 * Loading checks the tensor count and sizes and restores all of them into
 * the plan's bound inputs and state.  (The reference saves only the tensors
 * a caller passes, io/mod.rs:95-123; optimiser state is new.) */
int fg_plan_save(fg_plan *p, const char *path, int header);
int fg_plan_load(fg_plan *p, const char *path);
/* Human-readable launch list ("forward: gemm NN 64x256x784 bias+relu ...")
 * written to buf (truncated to len); *needed receives the full length. */
int fg_plan_describe(const fg_plan *p, char *buf, size_t len, size_t *needed);

/* ----------------------------------------------------- synthetic data */
/* Counter-based SplitMix64 generator keyed by (seed, tensor_id): element i
 * depends only on (seed, tensor_id, i), so host and device fills of the same
 * key produce the same values.  Used to build identical CPU/GPU inputs.
 *   uniform: [lo, hi) from the top 24 bits of the 64-bit draw
 *   normal : mean + std * Box-Muller(draws 2i, 2i+1), computed in double
 *   int    : floor(u32 * n / 2^32) in [0, n)                               */
int fg_rng_uniform_host(uint64_t seed, uint64_t tensor_id, float lo, float hi,
                        float *dst, uint64_t n);
int fg_rng_normal_host(uint64_t seed, uint64_t tensor_id, float mean, float std,
                       float *dst, uint64_t n);
int fg_rng_int_host(uint64_t seed, uint64_t tensor_id, uint32_t bound,
                    uint32_t *dst, uint64_t n);
int fg_rng_uniform_dev(fg_ctx *ctx, uint64_t seed, uint64_t tensor_id, float lo,
                       float hi, float *d_dst, uint64_t n);
int fg_rng_normal_dev(fg_ctx *ctx, uint64_t seed, uint64_t tensor_id, float mean,
                      float std, float *d_dst, uint64_t n);
int fg_rng_int_dev(fg_ctx *ctx, uint64_t seed, uint64_t tensor_id, uint32_t bound,
                   uint32_t *d_dst, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif /* FERROGRAD_HIP_H */
