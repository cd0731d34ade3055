// k_gemm16.hip -- host dispatch of the 16-bit (bf16 / fp16) MFMA GEMM:
// argument checks, alignment decisions and the tile-configuration choice.
// The kernel is in fg_gemm16_kernel.h, instantiated in k_gemm16_{bf16,f16}.hip.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "fg_gemm16_kernel.h"
#include "fg_internal.h"

namespace {

using fg::gemm16::Args;

// Pipelined whole-tile kernel on (1) or off (0): a knob for measurement builds.
#ifndef FG_GEMM16_PIPE
#define FG_GEMM16_PIPE 1
#endif
constexpr bool kPipe16 = FG_GEMM16_PIPE != 0;

int tiles(int M, int N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

// Tile configuration (indices as in fg_gemm16_kernel.h), from a measured
// sweep on MI355X of every configuration of the pipelined kernel (TFLOP/s,
// bf16, N(0,1) operands; fp16 within a few percent):
//  * squares that give >= one 256x256 tile per CU: 256x256 with 8 waves and
//    BK 64, direct loads, every layout: 1134-1162 / 1141-1171 / 1117-1145
//    (NN / NT / TN) at 4096^3 and 995-1003 for the 4096x4096x2048 weight
//    gradient, against 1115-1145 / 1143-1171 / 1117-1151 and 938-947 for
//    the staged BK 32 tile, and 1070-1098 / 1075-1105 / 1050-1080 and 839-846
//    for 4 waves (one per SIMD: each wave's waits idle its matrix unit).
//    The direct loads are issued as inline assembly (lds_dma16): as builtins
//    the compiler made every transposing LDS read wait for all of them in
//    flight (933 / 714 / 600 then);
//  * else 256x128 with 8 waves and BK 64 down to a quarter tile per CU: 956
//    for the 2048x4096x4096 forward, 799-855 for its NT data gradient, 302
//    for the 1000-wide head, where every smaller tile measured lower;
//  * else 128x128, else 64x64.
// The BK 64 tiles need K % 64 == 0; when only K % 32 == 0 holds, 256x256
// with 8 waves and BK 32 or 128x128 keep the pipelined kernel.  Other K take
// the 256x128 8-wave tiles where they give a quarter tile per CU: pipelined
// with a K tail (plan16), or gemm16_mfma where the operands do not allow it.
int pick_cfg16(int layout, int M, int N, int K, int cus) {
    if (K % 64 == 0) {
        if (tiles(M, N, 256, 256) >= cus) return 6;
        if (tiles(M, N, 256, 128) >= cus / 4) return 8;
    } else if (K % 32 == 0) {
        if (tiles(M, N, 256, 256) >= cus) return 1;
    } else if (tiles(M, N, 256, 128) >= cus / 4) {
        return 8;  // gemm16_mfma: 529 against 453 for 128x128 (2048x4096x1000 NT)
    }
    if (tiles(M, N, 128, 128) >= cus / 4) return 2;
    return 3;
}

// K slices for a pipelined GEMM whose output tiles fill at most half the
// CUs (the 1000-wide head and the 1024-wide layer's data gradient of a
// batch-2048 MLP: 64 tiles of 256x128): enough slices to give every CU a
// workgroup, each of whole K tiles and at least four of them.  Returns the
// number of slices (1: no split) and their depth in ks.
int split16(int cus, int M, int N, int K, int cfg, int &ks) {
    ks = 0;
    const int bk = fg::gemm16::cfg_bk16(cfg);
    // the configurations' tiles (fg_gemm16_kernel.h)
    const int bm = cfg == 2 ? 128 : cfg == 3 ? 64 : 256;
    const int bn = (cfg == 2 || cfg == 4 || cfg >= 7) ? 128 : cfg == 3 ? 64 : 256;
    const int t = tiles(M, N, bm, bn);
    if (2 * t > cus || K < 8 * bk) return 1;
    int s = std::min(cus / t, K / (4 * bk));
    if (s < 2) return 1;
    int k = (K + s - 1) / s;
    k = (k + bk - 1) / bk * bk;  // whole K tiles per slice
    s = (K + k - 1) / k;
    if (s < 2) return 1;
    ks = k;
    return s;
}

// The kernel choices of one call (operands as passed, colsum included).
struct Plan16 {
    bool vec = false, pipe = false;
    int cfg = 3, splits = 1, ks = 0;
};
Plan16 plan16(const fg_ctx *ctx, int layout, const Args &a) {
    Plan16 q;
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    // 16-byte operand loads need 16-byte aligned bases and leading
    // dimensions that keep every row start aligned (multiples of 8
    // elements); the bounds checks split per 8-element vector, so the
    // extents themselves are free.
    auto al = [](const void *p, unsigned m) { return (((uintptr_t)p) & (m - 1)) == 0; };
    q.vec = al(a.A, 16) && al(a.B, 16) && a.lda % 8 == 0 && a.ldb % 8 == 0;
#ifdef FG_GEMM16_FORCE_CFG  // tuning builds: one tile configuration for every shape
    q.cfg = FG_GEMM16_FORCE_CFG;
#else
    q.cfg = pick_cfg16(layout, a.M, a.N, a.K, cus);
#endif
    // The pipelined kernel: whole K tiles, 16-byte chunks of 8 elements along
    // each row-contiguous operand's rows (B of NN / TN, A of TN).
    const bool rc_ok = (layout == FG_NT || a.N % 8 == 0) && (layout != FG_TN || a.M % 8 == 0);
    q.pipe = kPipe16 && q.vec && rc_ok && a.K > 0 && a.K % fg::gemm16::cfg_bk16(q.cfg) == 0 &&
             a.M >= 8 && a.N >= 8 && q.cfg != 3;
    // K not a multiple of 32 on the 256x128 8-wave tiles (the 1000-deep data
    // gradient of a 1000-wide head): the pipelined kernel over the whole
    // tiles with the K tail from global memory, where each k-contiguous
    // operand's rows hold whole 8-element chunks of k (K % 8 == 0).
    if (!q.pipe && q.cfg == 8 && kPipe16 && q.vec && rc_ok && a.K > 0 && a.M >= 8 && a.N >= 8 &&
        (layout == FG_TN || a.K % 8 == 0)) {
        q.pipe = true;
        q.cfg = fg::gemm16::kCfgKTail16;
    }
    // Few tiles and a long K: K slices into the context's workspace when
    // what is reserved holds them (it is never grown for this), summed by a
    // second kernel in slot order -- deterministic, within the GEMM
    // tolerance of the unsplit sum.  With the fused column sums each slice
    // also leaves N fp32 sums, after the output slots.
    if (q.pipe && ctx->ws) {
        int ks;
        const int sl = split16(cus, a.M, a.N, a.K, q.cfg, ks);
        const uint64_t need = (uint64_t)sl * ((uint64_t)a.M * a.N + (a.colsum ? a.N : 0));
        if (sl > 1 && need * sizeof(float) <= ctx->ws_bytes) {
            q.splits = sl;
            q.ks = ks;
        }
    }
    return q;
}

// Argument checks of one call with M, N > 0 (nothing launched).
int gemm16_check(fg_ctx *ctx, int dtype, int layout, const Args &a, const char *who) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "%s: ctx is NULL", who);
    FG_REQUIRE(dtype == FG_DTYPE_F16 || dtype == FG_DTYPE_BF16, FG_ERR_UNSUPPORTED,
               "%s: dtype %d is not a 16-bit type (use fg_gemm_f32 for fp32)", who, dtype);
    FG_REQUIRE(a.M > 0 && a.N > 0 && a.K >= 0, FG_ERR_SHAPE, "%s: empty or negative shape", who);
    FG_REQUIRE(a.act >= 0 && a.act <= 2, FG_ERR_INVALID_ARGUMENT, "%s: bad act %d", who, a.act);
    FG_REQUIRE(a.A && a.B && a.C, FG_ERR_INVALID_ARGUMENT, "%s: NULL operand", who);
    const int a_cols = layout == FG_TN ? a.M : a.K;
    const int b_cols = layout == FG_NT ? a.K : a.N;
    FG_REQUIRE(a.lda >= std::max(a_cols, 1) && a.ldb >= std::max(b_cols, 1) && a.ldc >= a.N,
               FG_ERR_SHAPE, "%s: leading dimension too small", who);
    return FG_OK;
}

// 8-byte epilogue I/O where C / Z / bias allow it.
void set_vec_out(Args &a) {
    auto al = [](const void *q, unsigned m) { return (((uintptr_t)q) & (m - 1)) == 0; };
    a.vec_out = al(a.C, 8) && a.ldc % 4 == 0 && (!a.Z || (al(a.Z, 8) && a.ldz % 4 == 0)) &&
                (!a.bias || al(a.bias, 8));
}

int gemm16_common(fg_ctx *ctx, int dtype, int layout, Args &a, const char *who) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "%s: ctx is NULL", who);
    FG_REQUIRE(dtype == FG_DTYPE_F16 || dtype == FG_DTYPE_BF16, FG_ERR_UNSUPPORTED,
               "%s: dtype %d is not a 16-bit type (use fg_gemm_f32 for fp32)", who, dtype);
    FG_REQUIRE(layout >= FG_NN && layout <= FG_TN, FG_ERR_INVALID_ARGUMENT, "%s: bad layout %d",
               who, layout);
    FG_REQUIRE(a.M >= 0 && a.N >= 0 && a.K >= 0, FG_ERR_SHAPE, "%s: negative dimension", who);
    FG_REQUIRE(a.act >= 0 && a.act <= 2, FG_ERR_INVALID_ARGUMENT, "%s: bad act %d", who, a.act);
    FG_REQUIRE(!a.colsum || layout == FG_TN, FG_ERR_INVALID_ARGUMENT,
               "%s: column sums need the TN layout", who);
    if (a.N == 0) return FG_OK;
    if (a.M == 0) {  // no output rows, but the column sums of B still run
        if (!a.colsum) return FG_OK;
        FG_REQUIRE(a.B && a.ldb >= a.N, FG_ERR_INVALID_ARGUMENT, "%s: bad B", who);
        return fg_bias_grad(ctx, dtype, a.K, a.N, a.B, a.ldb, a.colsum, a.colsum_accumulate);
    }
    FG_REQUIRE(a.A && a.B && a.C, FG_ERR_INVALID_ARGUMENT, "%s: NULL operand", who);
    const int a_cols = layout == FG_TN ? a.M : a.K;
    const int b_cols = layout == FG_NT ? a.K : a.N;
    FG_REQUIRE(a.lda >= std::max(a_cols, 1) && a.ldb >= std::max(b_cols, 1) && a.ldc >= a.N,
               FG_ERR_SHAPE, "%s: leading dimension too small (lda=%d ldb=%d ldc=%d)", who, a.lda,
               a.ldb, a.ldc);
    FG_HIP(hipSetDevice(ctx->device));
    uint16_t *colsum = a.colsum;  // the bias gradient of fg_gemm_dw_x16, if any
    if (a.K == 0) a.A = a.B;  // loads are all masked; K=0 yields the epilogue of zero
    set_vec_out(a);
    const Plan16 q = plan16(ctx, layout, a);
    // Only the pipelined kernel sums B's columns; elsewhere the separate
    // reduction runs after the GEMM (same result up to the order of the
    // fp32 sums).
    if (colsum && !q.pipe) a.colsum = nullptr;
    a.partial = q.splits > 1 ? static_cast<float *>(ctx->ws) : nullptr;
    a.ksplit = q.splits > 1 ? q.ks : 0;
    a.colsum_partial =
        q.splits > 1 && a.colsum ? a.partial + (size_t)q.splits * a.M * a.N : nullptr;
    if (dtype == FG_DTYPE_BF16)
        fg::gemm16::launch_bf16(layout, a, q.vec, q.pipe, q.cfg, ctx->stream);
    else
        fg::gemm16::launch_f16(layout, a, q.vec, q.pipe, q.cfg, ctx->stream);
    FG_LAUNCH_CHECK(who);
    if (colsum && !q.pipe)
        return fg_bias_grad(ctx, dtype, a.K, a.N, a.B, a.ldb, colsum, a.colsum_accumulate);
    return FG_OK;
}

// A layer's dW (TN, with the fused column sums) and dX (NT, act' of Zs)
// arguments, as fg_gemm_dw_x16 and fg_gemm_bwd_x16 take them.
Args dw_args16(int M, int N, int K, const void *A, int lda, const void *B, int ldb, void *C,
               int ldc, int acc, void *colsum, int colsum_acc) {
    Args a{};
    a.A = static_cast<const uint16_t *>(A);
    a.B = static_cast<const uint16_t *>(B);
    a.C = static_cast<uint16_t *>(C);
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.act = FG_ACT_NONE;
    a.mode = 0;
    a.accumulate = acc ? 1 : 0;
    a.colsum = static_cast<uint16_t *>(colsum);
    a.colsum_accumulate = colsum_acc ? 1 : 0;
    return a;
}
Args dx_args16(int M, int N, int K, const void *A, int lda, const void *B, int ldb, int act,
               const void *Zs, int ldzs, void *C, int ldc, int acc) {
    Args a{};
    a.A = static_cast<const uint16_t *>(A);
    a.B = static_cast<const uint16_t *>(B);
    a.C = static_cast<uint16_t *>(C);
    a.Zs = static_cast<const uint16_t *>(Zs);
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.ldzs = ldzs;
    a.act = act;
    a.mode = 1;
    a.accumulate = acc ? 1 : 0;
    return a;
}
// Both pipelined on the pair's configurations, neither split.
bool pairable16(fg_ctx *ctx, Args &w, Args &x) {
    if (w.M <= 0 || w.N <= 0 || w.K <= 0 || x.M <= 0 || x.N <= 0 || x.K <= 0) return false;
    set_vec_out(w);
    set_vec_out(x);
    const Plan16 qw = plan16(ctx, FG_TN, w), qx = plan16(ctx, FG_NT, x);
    return qw.pipe && qx.pipe && qw.splits == 1 && qx.splits == 1 &&
           qw.cfg == fg::gemm16::kPair16CfgW && qx.cfg == fg::gemm16::kPair16CfgX;
}

}  // namespace

namespace fg {
// A layer's two gradient GEMMs with 16-bit tensors: one launch
// (gemm16_pair_big) when both take the large tiles' pipelined kernels
// unsplit, else fg_gemm_dw_x16 then fg_gemm_bwd_x16.  Each part runs
// exactly as its own call.
int gemm16_dw_dx(fg_ctx *ctx, int dtype, int M1, int N1, int K1, const void *A1, int lda1,
                 const void *B1, int ldb1, void *C1, int ldc1, int acc1, void *colsum,
                 int colsum_acc, int M2, int N2, int K2, const void *A2, int lda2,
                 const void *B2, int ldb2, int act, const void *Zs, int ldzs, void *C2, int ldc2,
                 int acc2) {
    Args w = dw_args16(M1, N1, K1, A1, lda1, B1, ldb1, C1, ldc1, acc1, colsum, colsum_acc);
    Args x = dx_args16(M2, N2, K2, A2, lda2, B2, ldb2, act, Zs, ldzs, C2, ldc2, acc2);
    const bool checked = M1 > 0 && N1 > 0 && M2 > 0 && N2 > 0 &&
                         gemm16_check(ctx, dtype, FG_TN, w, "fg_gemm_dw_x16") == FG_OK &&
                         gemm16_check(ctx, dtype, FG_NT, x, "fg_gemm_bwd_x16") == FG_OK &&
                         (act == FG_ACT_NONE || (Zs && ldzs >= N2));
    if (!checked || !pairable16(ctx, w, x)) {
        fg::clear_error();  // the calls below report any error themselves
        const int rc = fg_gemm_dw_x16(ctx, dtype, M1, N1, K1, A1, lda1, B1, ldb1, C1, ldc1, acc1,
                                      colsum, colsum_acc);
        if (rc) return rc;
        return fg_gemm_bwd_x16(ctx, dtype, FG_NT, M2, N2, K2, A2, lda2, B2, ldb2, act, Zs, ldzs,
                               C2, ldc2, acc2);
    }
    FG_HIP(hipSetDevice(ctx->device));
    if (dtype == FG_DTYPE_BF16)
        fg::gemm16::launch_pair_bf16(w, x, ctx->stream);
    else
        fg::gemm16::launch_pair_f16(w, x, ctx->stream);
    FG_LAUNCH_CHECK("gemm16_dw_dx");
    return FG_OK;
}

// Dispatches of gemm16_dw_dx for these operands (no launch).
int gemm16_dw_dx_dispatches(fg_ctx *ctx, int M1, int N1, int K1, const void *A1, int lda1,
                            const void *B1, int ldb1, int M2, int N2, int K2, const void *A2,
                            int lda2, const void *B2, int ldb2) {
    const int sep = gemm16_dispatches(ctx, FG_TN, M1, N1, K1, A1, lda1, B1, ldb1, true) +
                    gemm16_dispatches(ctx, FG_NT, M2, N2, K2, A2, lda2, B2, ldb2, false);
    if (!ctx) return sep;
    void *c = reinterpret_cast<void *>(256);  // only the operands' alignment enters the choice
    Args w = dw_args16(M1, N1, K1, A1, lda1, B1, ldb1, c, N1, 0, c, 0);
    Args x = dx_args16(M2, N2, K2, A2, lda2, B2, ldb2, FG_ACT_NONE, nullptr, 0, c, N2, 0);
    return pairable16(ctx, w, x) ? 1 : sep;
}

// Dispatches of one 16-bit GEMM call with these operands (no launch): the
// GEMM, its summing kernel when it splits K, the column-sum reduction's two
// when colsum is asked off the pipelined kernel.
int gemm16_dispatches(fg_ctx *ctx, int layout, int M, int N, int K, const void *A, int lda,
                      const void *B, int ldb, bool colsum) {
    if (!ctx || M <= 0 || N <= 0 || K <= 0) return 1;
    Args a{};
    a.A = static_cast<const uint16_t *>(A);
    a.B = static_cast<const uint16_t *>(B);
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.colsum = colsum ? reinterpret_cast<uint16_t *>(256) : nullptr;
    const Plan16 q = plan16(ctx, layout, a);
    if (colsum && !q.pipe) return 3;
    return q.splits > 1 ? 2 : 1;
}

// Workspace bytes a 16-bit GEMM of this shape splits K into when the
// workspace holds them (0: it does not split), for planners that size a
// workspace ahead.  Assumes the pipelined kernel (aligned operands).
uint64_t gemm16_split_ws_bytes(int cus, int layout, int M, int N, int K, bool colsum) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    cus = cus > 0 ? cus : 256;
    const int cfg = pick_cfg16(layout, M, N, K, cus);
    if (cfg == 3 || K % fg::gemm16::cfg_bk16(cfg) != 0) return 0;
    int ks;
    const int sl = split16(cus, M, N, K, cfg, ks);
    return sl > 1 ? (uint64_t)sl * ((uint64_t)M * N + (colsum ? N : 0)) * sizeof(float) : 0;
}
}  // namespace fg

FG_API int fg_gemm_x16(fg_ctx *ctx, int dtype, int layout, int M, int N, int K, const void *d_A,
                       int lda, const void *d_B, int ldb, const void *d_bias, int act, void *d_C,
                       int ldc, void *d_Z, int ldz, int accumulate) {
    Args a{};
    a.A = static_cast<const uint16_t *>(d_A);
    a.B = static_cast<const uint16_t *>(d_B);
    a.C = static_cast<uint16_t *>(d_C);
    a.Z = static_cast<uint16_t *>(d_Z);
    a.bias = static_cast<const uint16_t *>(d_bias);
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.ldz = d_Z ? ldz : 0;
    a.act = act;
    a.mode = 0;
    a.accumulate = accumulate ? 1 : 0;
    FG_REQUIRE(!d_Z || ldz >= N, FG_ERR_SHAPE, "fg_gemm_x16: ldz=%d < N=%d", ldz, N);
    FG_REQUIRE(!(accumulate && act != FG_ACT_NONE), FG_ERR_INVALID_ARGUMENT,
               "fg_gemm_x16: accumulate requires act NONE");
    return gemm16_common(ctx, dtype, layout, a, "fg_gemm_x16");
}

FG_API int fg_gemm_dw_x16(fg_ctx *ctx, int dtype, int M, int N, int K, const void *d_A, int lda,
                          const void *d_B, int ldb, void *d_C, int ldc, int accumulate,
                          void *d_colsum, int colsum_accumulate) {
    Args a{};
    a.A = static_cast<const uint16_t *>(d_A);
    a.B = static_cast<const uint16_t *>(d_B);
    a.C = static_cast<uint16_t *>(d_C);
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.act = FG_ACT_NONE;
    a.mode = 0;
    a.accumulate = accumulate ? 1 : 0;
    a.colsum = static_cast<uint16_t *>(d_colsum);
    a.colsum_accumulate = colsum_accumulate ? 1 : 0;
    return gemm16_common(ctx, dtype, FG_TN, a, "fg_gemm_dw_x16");
}

FG_API int fg_gemm_bwd_x16(fg_ctx *ctx, int dtype, int layout, int M, int N, int K,
                           const void *d_A, int lda, const void *d_B, int ldb, int act,
                           const void *d_Zs, int ldzs, void *d_C, int ldc, int accumulate) {
    Args a{};
    a.A = static_cast<const uint16_t *>(d_A);
    a.B = static_cast<const uint16_t *>(d_B);
    a.C = static_cast<uint16_t *>(d_C);
    a.Zs = static_cast<const uint16_t *>(d_Zs);
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.ldzs = ldzs;
    a.act = act;
    a.mode = 1;
    a.accumulate = accumulate ? 1 : 0;
    FG_REQUIRE(act == FG_ACT_NONE || (d_Zs && ldzs >= N), FG_ERR_INVALID_ARGUMENT,
               "fg_gemm_bwd_x16: act %d needs Zs with ldzs >= N", act);
    return gemm16_common(ctx, dtype, layout, a, "fg_gemm_bwd_x16");
}

FG_API int fg_matmul_bwd_x16(fg_ctx *ctx, int dtype, int M, int N, int K, const void *d_X,
                             int ldx, const void *d_W, int ldw, const void *d_dZ, int lddz,
                             int act, const void *d_Zs, int ldzs, void *d_dX, int lddx,
                             void *d_dW, int lddw, void *d_dbias, int accumulate) {
    const char *who = "fg_matmul_bwd_x16";
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "%s: ctx is NULL", who);
    FG_REQUIRE(act >= FG_ACT_NONE && act <= FG_ACT_GELU, FG_ERR_INVALID_ARGUMENT,
               "%s: bad act %d", who, act);
    FG_REQUIRE(M >= 0 && N >= 0 && K >= 0, FG_ERR_SHAPE, "%s: negative dimension", who);
    FG_REQUIRE(d_X && d_W && d_dZ && d_dX && d_dW, FG_ERR_INVALID_ARGUMENT,
               "%s: NULL operand or output", who);
    FG_REQUIRE(ldx >= K && ldw >= N && lddz >= N && lddx >= K && lddw >= N,
               FG_ERR_INVALID_ARGUMENT, "%s: a leading dimension is below its row length", who);
    FG_REQUIRE(act == FG_ACT_NONE || (d_Zs && ldzs >= K), FG_ERR_INVALID_ARGUMENT,
               "%s: act %d needs Zs with ldzs >= K", who, act);
    // dW: TN K x N over M; dX: NT M x K over N.
    return fg::gemm16_dw_dx(ctx, dtype, K, N, M, d_X, ldx, d_dZ, lddz, d_dW, lddw, accumulate,
                            d_dbias, accumulate, M, K, N, d_dZ, lddz, d_W, ldw, act, d_Zs, ldzs,
                            d_dX, lddx, accumulate);
}
