// fg_internal.h -- shared internals of the gfx950 backend (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/ferrograd_hip.h"

namespace fg {

// Thread-local last error (fg_last_error_msg).
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Map a HIP status to an fg_status and record the message.  Mirrors the
// HipError -> ErrorKind mapping of rocm/mod.rs:468-545.
int hip_fail(hipError_t e, const char *what, const char *file, int line);

}  // namespace fg

struct fg_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    int cu_count = 0;
    char arch[64] = {0};
    // Scratch workspace for direct kernel calls that need partial results.
    // Grown by fg::workspace(); a workspace it replaces stays allocated in
    // ws_retired until fg_ctx_destroy, because a graph captured earlier may
    // still hold its address.
    void *ws = nullptr;
    uint64_t ws_bytes = 0;
    std::vector<void *> ws_retired;
    // Set on a plan's own view of its context: ws is a fixed part of the
    // plan's arena and fg::workspace() never replaces it.
    bool ws_fixed = false;
    // The planner's captured steps: with defer_reduce set, the next split-K
    // summing launch is not launched but held here (its GemmArgs and slice
    // count), for the optimiser launch that follows to run beside its own
    // work (fg::sgd_step_with_pending) or to launch first.
    bool defer_reduce = false;
    int pending_splits = 0;
    alignas(16) unsigned char pending[256];
    // A mean loss left by a loss finished in the head GEMM (captured steps):
    // mean_dst = mean of mean_rows row losses at mean_src, for the optimiser
    // launch to compute (or fg::launch_pending_mean).
    const float *mean_src = nullptr;
    float *mean_dst = nullptr;
    int mean_rows = 0;
};

struct fg_buf {
    int device = 0;
    void *ptr = nullptr;
    uint64_t bytes = 0;
};

namespace fg {
// A captured step's softmax + CE loss finished by the skinny head GEMM that
// computes its logits (fg_gemm_skinny.h, fg_softmax_row.h): labels, and
// where it writes (probs may be NULL).  The mean is left to a later launch.
struct CeOut {
    const uint32_t *labels;
    float *row_loss;
    float *dlogits;
    float *probs;
    int ldd, ldp;
    float scale;
    // Optionally the head's data gradient as well (fp32 dlogits only):
    // dz = (dlogits . B^T) * act'(Z of the summed GEMM) for the kernel's
    // rows, with the MFMA sequence of the 64x64 tile kernels, so the same
    // bits as the backward's own NT GEMM; NULL: none.
    float *dz;
    int lddz;
    int dz_act;
};

// [begin, end) of device memory, as addresses.
struct ByteRange {
    uintptr_t begin, end;
    bool overlaps(const ByteRange &o) const {
        return begin < end && o.begin < o.end && begin < o.end && o.begin < end;
    }
};

// The held split-K summing launch (fg_ctx::pending, k_gemm.hip): its block
// count for M x N outputs, a launch of it alone (clears it), and the memory
// it writes (C) and reads besides its slices (act' operand, bias).
int reduce_blocks(const fg_ctx *ctx, int M, int N);
int launch_pending_reduce(fg_ctx *ctx);
void pending_reduce_ranges(const fg_ctx *ctx, ByteRange out[3]);
// The held mean loss (fg_ctx::mean_*) in a launch of its own; clears it.
int launch_pending_mean(fg_ctx *ctx);
// SGD over `mt` with the summing launch and / or the mean loss held in
// `held` (a plan's context view) run by extra workgroups of the same launch
// (k_gemm.hip); the caller has checked that the held summing pass and the
// SGD update touch disjoint memory.  Clears what it runs.
int sgd_step_with_pending(fg_ctx *ctx, fg_mt *mt, float lr, int zero_grad, fg_ctx *held);

// Returns a workspace pointer of at least `bytes`, or nullptr with the error
// set.  A context's workspace grows by allocating a larger one; the old one
// is retired, not freed (captured graphs may use it).  A fixed workspace (a
// plan's) never grows: a request beyond it fails.
void *workspace(fg_ctx *ctx, uint64_t bytes);

// Looks up the device address of the fixed scratch array of
// fg_bias_grad_noalloc on `device` (current), once per device (k_noalloc.hip).
int noalloc_init(int device);

// Bytes of workspace fg_bias_grad needs for an M x N reduction on a device
// with `cus` compute units (the partial sums of its row splits).
uint64_t bias_grad_ws_bytes(int cus, int M, int N);
// Workspace bytes of the K slices a 16-bit GEMM of this shape takes when the
// workspace holds them (0: no split); colsum: with the fused column sums.
uint64_t gemm16_split_ws_bytes(int cus, int layout, int M, int N, int K, bool colsum);
// Dispatches of one 16-bit GEMM call (no launch; colsum: the fused bias
// gradient of fg_gemm_dw_x16 is asked).
int gemm16_dispatches(fg_ctx *ctx, int layout, int M, int N, int K, const void *A, int lda,
                      const void *B, int ldb, bool colsum);
// A layer's dW (TN, fused column sums) and dX (NT, act') with 16-bit tensors,
// in one launch when their kernels pair; its dispatches (no launch).
int gemm16_dw_dx(fg_ctx *ctx, int dtype, int M1, int N1, int K1, const void *A1, int lda1,
                 const void *B1, int ldb1, void *C1, int ldc1, int acc1, void *colsum,
                 int colsum_acc, int M2, int N2, int K2, const void *A2, int lda2,
                 const void *B2, int ldb2, int act, const void *Zs, int ldzs, void *C2, int ldc2,
                 int acc2);
int gemm16_dw_dx_dispatches(fg_ctx *ctx, int M1, int N1, int K1, const void *A1, int lda1,
                            const void *B1, int ldb1, int M2, int N2, int K2, const void *A2,
                            int lda2, const void *B2, int ldb2);

// Adam with device-resident step counter / bias-correction scalars
// (k_optim.hip).  d_state points at adam_dev_state_bytes() zeroed bytes.
uint64_t adam_dev_state_bytes();
int mt_adam_dev(fg_ctx *ctx, fg_mt *mt, float lr, float b1, float b2, float eps, void *d_state,
                int zero_grad);
// The two halves of mt_adam_dev, for updates split over several launches
// (and streams) within one step: one advance, then any number of updates.
// max_blocks (0: one workgroup per chunk) caps the grid; each workgroup then
// walks several chunks.
int adam_dev_advance(fg_ctx *ctx, float lr, float b1, float b2, void *d_state);
int adam_dev_advance_on(hipStream_t stream, float lr, float b1, float b2, void *d_state);
int mt_adam_dev_update(fg_mt *mt, hipStream_t stream, float b1, float b2, float eps,
                       const void *d_state, int zero_grad, uint32_t max_blocks);

// fg_softmax_ce with one more output: probs[r][c] = softmax(x_r)[c] (ld
// ldp, element type dtype; NULL: none), so a fused loss launch can also
// produce the forward's softmax output (k_softmax.hip).
int softmax_ce_ex(fg_ctx *ctx, int dtype, const void *d_logits, int ldx, const uint32_t *d_labels,
                  int R, int C, float grad_scale, float *d_row_loss, float *d_mean_loss,
                  void *d_dlogits, int ldd, uint32_t *d_argmax, void *d_probs, int ldp);

// The mean loss of R per-row losses, on `stream`, by the kernel softmax_ce_ex
// launches for it (same operations, so the same bits).
int launch_mean_loss(hipStream_t stream, const float *d_row_loss, int R, float *d_mean_loss);

// Kernel dispatches of softmax_ce_ex for R x C (with or without the mean).
int softmax_ce_dispatches(int R, int C, bool mean);
// R x C takes the 16-lane row kernel (fg_softmax_row.h), whose row code the
// skinny head GEMM can run in a captured step.
bool softmax_ce_row16_case(int R, int C);

// Elementwise program launch (k_eltwise_prog.hip): through its compiled
// kernel or the interpreter; prepare_eltwise compiles the kernel a launch
// would take, ahead of a stream capture.
struct EltProgram;
int launch_eltwise(fg_ctx *ctx, const EltProgram &p);
int prepare_eltwise(fg_ctx *ctx, const EltProgram &p);
// Compiled elementwise kernels (fg_elt_jit.cpp): whether the mode selects
// one for p; the compile / launch of a validated program (`live`: values
// kept at once; *launched false when the interpreter is to run it); the
// interpreter's launch count.
bool eltwise_jit_selected(const EltProgram &p);
int eltwise_jit(fg_ctx *ctx, const EltProgram &p, int live, bool prepare_only, bool *launched);
void eltwise_count_interpreted();
// Kernel dispatches of one fp32 GEMM call with these operands (2 when K is
// split: the slices, then the summing epilogue), for plan descriptions.
int gemm_f32_dispatches(fg_ctx *ctx, int layout, int M, int N, int K, const void *A, int lda,
                        const void *B, int ldb, bool colsum);
// A layer's dW (TN, fused column sums) and dX (NT, act'(Zs)) GEMMs, in one
// launch when both take small kernels (k_gemm.hip), and its dispatch count.
int gemm_dw_dx_f32(fg_ctx *ctx, int M1, int N1, int K1, const float *A1, int lda1,
                   const float *B1, int ldb1, float *C1, int ldc1, int acc1, float *colsum,
                   int colsum_acc, int M2, int N2, int K2, const float *A2, int lda2,
                   const float *B2, int ldb2, int act, const float *Zs, int ldzs, float *C2,
                   int ldc2, int acc2);
int gemm_dw_dx_dispatches(fg_ctx *ctx, int M1, int N1, int K1, const void *A1, int lda1,
                          const void *B1, int ldb1, int M2, int N2, int K2, const void *A2,
                          int lda2, const void *B2, int ldb2);
// The skinny kernel's largest N (output columns).
int gemm_skinny_max_n();
// A small head's dW (+ dbias, TN) beside a layer's dW and dX, in one launch
// when the head's takes the skinny kernel and the two pair (k_gemm.hip);
// and its dispatch count.
int gemm_dw_dw_dx_f32(fg_ctx *ctx, int M0, int N0, int K0, const float *A0, int lda0,
                      const float *B0, int ldb0, float *C0, int ldc0, int acc0, float *colsum0,
                      int colsum_acc0, int M1, int N1, int K1, const float *A1, int lda1,
                      const float *B1, int ldb1, float *C1, int ldc1, int acc1, float *colsum1,
                      int colsum_acc1, int M2, int N2, int K2, const float *A2, int lda2,
                      const float *B2, int ldb2, int act, const float *Zs, int ldzs, float *C2,
                      int ldc2, int acc2);
int gemm_dw_dw_dx_dispatches(fg_ctx *ctx, int M0, int N0, int K0, const void *A0, int lda0,
                             const void *B0, int ldb0, int M1, int N1, int K1, const void *A1,
                             int lda1, const void *B1, int ldb1, int M2, int N2, int K2,
                             const void *A2, int lda2, const void *B2, int ldb2);
// Two forward GEMMs in a row, the second (NN) reading the first's output as
// its A operand: when the first splits K and the second takes the skinny
// kernel, the second sums the first's slices (k_gemm.hip); and the dispatch
// count of that call.
// With `ce` (a loss over the second GEMM's output, at most 16 columns and
// 1024 rows, no accumulation) the chained kernel also finishes that loss and
// *ce_done is set; otherwise *ce_done stays false and the caller runs it.
int gemm_fwd_chain_f32(fg_ctx *ctx, int M1, int N1, int K1, const float *A1, int lda1,
                       const float *B1, int ldb1, const float *bias1, int act1, float *C1,
                       int ldc1, float *Z1, int ldz1, int M2, int N2, int K2, const float *A2,
                       int lda2, const float *B2, int ldb2, const float *bias2, int act2,
                       float *C2, int ldc2, float *Z2, int ldz2, int acc2,
                       const CeOut *ce = nullptr, bool *ce_done = nullptr);
int gemm_fwd_chain_dispatches(fg_ctx *ctx, int M1, int N1, int K1, const void *A1, int lda1,
                              const void *B1, int ldb1, const void *bias1, void *C1, int ldc1,
                              void *Z1, int ldz1, int M2, int N2, int K2, const void *A2, int lda2,
                              const void *B2, int ldb2);
}  // namespace fg

#define FG_HIP(call)                                                     \
    do {                                                                 \
        hipError_t fg_e_ = (call);                                       \
        if (fg_e_ != hipSuccess)                                         \
            return fg::hip_fail(fg_e_, #call, __FILE__, __LINE__);       \
    } while (0)

#define FG_REQUIRE(cond, code, ...)                                      \
    do {                                                                 \
        if (!(cond)) {                                                   \
            fg::set_error(__VA_ARGS__);                                  \
            return (code);                                               \
        }                                                                \
    } while (0)

// Check the launch that was just enqueued.
#define FG_LAUNCH_CHECK(name) FG_HIP(hipGetLastError())

#define FG_API extern "C" __attribute__((visibility("default")))
