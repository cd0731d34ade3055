// k_gemm.hip -- host dispatch of the MFMA GEMM (tile-configuration choice,
// argument checks) and the bias-gradient column reduction.  The kernel
// itself is in fg_gemm_kernel.h, instantiated per layout in k_gemm_*.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "fg_bias_grad.h"
#include "fg_gemm_kernel.h"
#include "fg_gemm_skinny.h"
#include "fg_half.h"
#include "fg_internal.h"
#include "fg_optim.h"
#include "fg_softmax_row.h"

namespace {

using fg::gemm::GemmArgs;
using fg::gemm::kThreads;
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ dispatch
// Tile configuration per call (indices as in fg_gemm_kernel.h), from a
// measured sweep of every configuration of the pipelined kernel on MI355X
// (256 CUs, N(0,1) operands, HIP events) over the BASELINE shapes, TFLOP/s:
//  * NN (forward): 256x256 with 8 waves for K >= 4096 squares that fill the
//    chip (138-145 at 4096^3, against 139-142 for the 256x128 tiles); else
//    256x128 with 8 waves when it yields >= one tile per CU (125 at
//    2048x4096x4096, 135 at K = 1024); else 128x64 (131 for the 1000-wide
//    head, against 70 for 128x128 on a quarter of the CUs); 64x64 for
//    anything smaller.
//  * NT (dA): 256x256 with 8 waves for large-K squares that fill the chip
//    (145 at 4096^3); else 256x128 with 8 waves when it gives >= one tile per
//    CU (137 at 2048x4096x4096); else 128x128 or 128x64 (137 for 128x64 at
//    2048x1024x4096, against 73 for 128x128).
//  * TN (dW): 256x256 with 8 waves whenever it fills the chip (143 at 4096^3;
//    141 at 4096x4096x2048, the c5 hidden dW, against 136.5 for 256x128 with
//    4 waves, with the interleaved fragments of the TN layout); 256x128 with
//    4 waves at >= two tiles per CU; then 128x64 at >= two tiles per CU
//    (131-133 for the 1024- and 1000-wide layers, against 125-127 for
//    128x128); else 128x128; else 128x64.
// K % BK != 0 (the 1000-deep head dA) takes the pipelined kernel's staged
// instances with a zero-filled last K tile (the 256x256 tiles give way to
// 256x128).
int tiles(int M, int N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

int pick_cfg(int layout, int M, int N, int K, int cus) {
    if (layout == FG_NN) {
        if (K >= 4096 && tiles(M, N, 256, 256) >= cus) return 6;
        if (tiles(M, N, 256, 128) >= cus) return 7;
        if (tiles(M, N, 128, 64) >= cus) return 5;
        return 4;
    }
    if ((K >= 4096 || layout == FG_TN) && tiles(M, N, 256, 256) >= cus) return 6;
    if (layout == FG_NT) {
        if (tiles(M, N, 256, 128) >= cus) return 7;
    } else {
        if (tiles(M, N, 256, 128) >= 2 * cus) return 1;
        if (tiles(M, N, 128, 64) >= 2 * cus) return 5;
    }
    if (tiles(M, N, 128, 128) >= cus) return 3;
    if (tiles(M, N, 128, 64) >= cus) return 5;
    return 4;
}

// Split-K epilogue: out[m][n] = epilogue(sum over the slots, in order, of
// partial[s][m][n]) -- the same per-element operations as the GEMM kernels'
// epilogue (fg_gemm_kernel.h epi_value), so bias / activation / Z / act' /
// accumulate behave alike.  Deterministic: the slot order is fixed.
__global__ __launch_bounds__(kThreads) void splitk_reduce(GemmArgs p, int splits) {
    fg::gemm::split_sum_blocks(p, splits, blockIdx.x, gridDim.x);
}

// SGD over a tensor list (workgroups below nchunks, one chunk each) and a
// held split-K summing pass (the rest) in one launch: independent work
// (the caller has checked that they touch disjoint memory), each part
// exactly as its own kernel does it.
// The last workgroup (with mean_dst) computes a held mean loss as the
// one-workgroup loss kernel would.
static_assert(fg::optim::kThreads == kThreads, "one block size for every part");
static_assert(kThreads >= fg::smrow::kSlots, "the mean's slots");
__global__ __launch_bounds__(kThreads) void sgd_and_split_sum(
    const fg::optim::MTTensor *__restrict__ tensors, const fg::optim::MTChunk *__restrict__ chunks,
    float lr, int zero_grad, int vec, uint32_t nchunks, GemmArgs red, int splits, uint32_t nred,
    const float *__restrict__ mean_src, int mean_rows, float *__restrict__ mean_dst) {
    __shared__ double sh[fg::smrow::kSlots];
    const uint32_t b = blockIdx.x;
    if (b < nchunks)
        fg::optim::sgd_chunk(tensors, chunks, lr, zero_grad, vec, b);
    else if (b < nchunks + nred)
        fg::gemm::split_sum_blocks(red, splits, b - nchunks, nred);
    else
        fg::smrow::mean_rows(mean_src, mean_rows, mean_dst, sh);
}

__global__ __launch_bounds__(kThreads) void mean_rows_kernel(const float *__restrict__ src, int R,
                                                             float *__restrict__ dst) {
    __shared__ double sh[fg::smrow::kSlots];
    fg::smrow::mean_rows(src, R, dst, sh);
}

// Split K over workgroup rows when the output gives few tiles (under half
// the CUs) and K is long (at least kSplitMinKTiles K tiles, and at least 4
// per slice; c1's K = 256 GEMMs, 16 K tiles, run 62 us per step split and
// 69 us unsplit, though unsplit saves two dispatches): each slice's raw
// product goes to the context's workspace, which must already hold them
// (every plan has its own of at least 1 MiB; direct callers reserve one with
// fg_ctx_reserve_workspace; it is never grown here, so launches stay
// capturable).  The fused column sum of fg_gemm_dw is not split.
// Returns the number of slices (1: no split).
#ifndef FG_SPLIT_MIN_KTILES  // tuning builds may set it
#define FG_SPLIT_MIN_KTILES 8
#endif
constexpr int kSplitMinKTiles = FG_SPLIT_MIN_KTILES;

int plan_split_k(fg_ctx *ctx, GemmArgs &a, int cfg, bool vec) {
    if (a.colsum || a.K <= 0) return 1;
    int bm, bn;
    fg::gemm::cfg_tile(cfg, vec, bm, bn);
    const int bk = vec ? fg::gemm::cfg_bk(cfg) : 16;
    if (a.K < kSplitMinKTiles * bk) return 1;
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    int s = std::min(cus / (2 * tiles(a.M, a.N, bm, bn)), a.K / (4 * bk));
    if (s < 2) return 1;
    int ks = (a.K + s - 1) / s;
    ks = (ks + bk - 1) / bk * bk;  // whole K tiles per slice
    s = (a.K + ks - 1) / ks;
    if (s < 2 || (uint64_t)s * a.M * a.N * sizeof(float) > ctx->ws_bytes) return 1;
    a.partial = static_cast<float *>(ctx->ws);
    a.ksplit = ks;
    return s;
}

// Skinny shapes (few columns, short K, at most one 16-row workgroup per CU)
// take the one-round-trip kernel of k_gemm_skinny.hip: c1's second layer
// (64x10x256) and its weight gradient with the bias gradient (TN 256x10x64).
bool use_skinny(fg_ctx *ctx, const GemmArgs &a, int pro) {
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    return pro == fg::gemm::kProNone && a.N <= fg::gemm::kSkinnyN && a.K > 0 &&
           a.K <= fg::gemm::kSkinnyK && (int64_t)a.M <= 16LL * cus;
}

// The kernel choices of one GEMM call (sets a.vec_out, and a.partial /
// a.ksplit when K is split): the skinny kernel (skinny; then nothing else
// applies), 16-byte operand loads (vec), the pipelined kernel (pipe) and
// whether its last K tile is partial (ktail), the tile configuration and the
// number of K slices.  pro: the prologue code (fg::gemm::kPro*), whose
// tensor Pz must meet the same 16-byte conditions as the operand it scales.
void plan_gemm(fg_ctx *ctx, int layout, GemmArgs &a, bool &skinny, bool &vec, bool &pipe,
               bool &ktail, int &cfg, int &splits, int pro = fg::gemm::kProNone) {
    skinny = use_skinny(ctx, a, pro);
    vec = pipe = ktail = false;
    cfg = 0;
    splits = 1;
    if (skinny) return;
    // The 16-byte path needs 16-byte aligned bases and every row start
    // aligned, i.e. leading dimensions and the contiguous extents that the
    // bounds checks split on (K for k-contiguous operands, M / N otherwise)
    // divisible by 4.
    const bool aligned_ptrs = ((((uintptr_t)a.A) | ((uintptr_t)a.B)) & 15u) == 0;
    vec = aligned_ptrs && a.lda % 4 == 0 && a.ldb % 4 == 0;
    if (layout == FG_NN) vec = vec && a.K % 4 == 0 && a.N % 4 == 0;
    if (layout == FG_NT) vec = vec && a.K % 4 == 0;
    if (layout == FG_TN) vec = vec && a.M % 4 == 0 && a.N % 4 == 0;
    if (pro != fg::gemm::kProNone) vec = vec && (((uintptr_t)a.Pz) & 15u) == 0 && a.ldp % 4 == 0;
#ifdef FG_GEMM_FORCE_CFG  // tuning builds: one tile configuration for every shape
    cfg = FG_GEMM_FORCE_CFG;
#else
    cfg = pick_cfg(layout, a.M, a.N, a.K, ctx->cu_count > 0 ? ctx->cu_count : 256);
#endif
    if (pro != fg::gemm::kProNone) cfg = fg::gemm::pro_cfg(cfg);
    auto al16 = [](const void *q) { return (((uintptr_t)q) & 15u) == 0; };
    a.vec_out = al16(a.C) && a.ldc % 4 == 0 && (!a.Z || (al16(a.Z) && a.ldz % 4 == 0)) &&
                (!a.bias || al16(a.bias));
    // The pipelined kernel's 16-byte tile loads need at least one 16-byte
    // chunk per row-contiguous operand row (edge chunks are clamped, not
    // masked).  A partial last K tile (K % BK != 0) is zero-filled by the
    // staged-tile instances (ktail); the prologue instances need whole tiles
    // and leave such shapes to gemm_f32_mfma.
    pipe = fg::gemm::kPipe && vec && a.K > 0 && a.M >= 4 && a.N >= 4;
    ktail = false;
    if (pipe && a.K % fg::gemm::cfg_bk(cfg) != 0) {
        if (pro != fg::gemm::kProNone) {
            pipe = false;
        } else {
            ktail = true;
            cfg = fg::gemm::pro_cfg(cfg);  // staged tiles
        }
    }
    splits = plan_split_k(ctx, a, cfg, vec);
}

// One GEMM call, validated and planned (gemm_prepare), then launched
// (gemm_launch): alone, or beside another in one launch (fg::gemm_dw_dx_f32).
struct Planned {
    GemmArgs a{};
    int layout = FG_NN, pro = fg::gemm::kProNone, cfg = 0, splits = 1;
    bool skinny = false, vec = false, pipe = false, ktail = false;
    bool empty = false;  // M == 0 or N == 0: nothing to launch
};

int gemm_prepare(fg_ctx *ctx, int layout, const GemmArgs &a0, const char *who, int pro,
                 Planned &P) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "%s: ctx is NULL", who);
    FG_REQUIRE(layout >= FG_NN && layout <= FG_TN, FG_ERR_INVALID_ARGUMENT, "%s: bad layout %d",
               who, layout);
    GemmArgs &a = P.a;
    a = a0;
    P.layout = layout;
    P.pro = pro;
    FG_REQUIRE(a.M >= 0 && a.N >= 0 && a.K >= 0, FG_ERR_SHAPE, "%s: negative dimension", who);
    FG_REQUIRE(a.act >= 0 && a.act <= 2, FG_ERR_INVALID_ARGUMENT, "%s: bad act %d", who, a.act);
    if (a.M == 0 || a.N == 0) {
        P.empty = true;
        return FG_OK;
    }
    FG_REQUIRE(a.A && a.B && a.C, FG_ERR_INVALID_ARGUMENT, "%s: NULL operand", who);
    // Leading dimensions: A is [M][K] (NN/NT) or [K][M] (TN); B is [K][N]
    // (NN/TN) or [N][K] (NT); C is [M][N].
    const int a_cols = layout == FG_TN ? a.M : a.K;
    const int b_cols = layout == FG_NT ? a.K : a.N;
    FG_REQUIRE(a.lda >= std::max(a_cols, 1) && a.ldb >= std::max(b_cols, 1) && a.ldc >= a.N,
               FG_ERR_SHAPE, "%s: leading dimension too small (lda=%d ldb=%d ldc=%d)", who, a.lda,
               a.ldb, a.ldc);
    FG_HIP(hipSetDevice(ctx->device));
    if (a.K == 0) a.A = a.B;  // loads are all masked; K=0 yields the epilogue of zero
    plan_gemm(ctx, layout, a, P.skinny, P.vec, P.pipe, P.ktail, P.cfg, P.splits, pro);
    return FG_OK;
}

void launch_reduce(fg_ctx *ctx, const GemmArgs &a, int splits) {
    if (ctx->defer_reduce) {  // held for the optimiser launch that follows
        static_assert(sizeof(GemmArgs) <= sizeof(ctx->pending), "pending summing launch");
        std::memcpy(ctx->pending, &a, sizeof a);
        ctx->pending_splits = splits;
        ctx->defer_reduce = false;
        return;
    }
    splitk_reduce<<<fg::reduce_blocks(ctx, a.M, a.N), kThreads, 0, ctx->stream>>>(a, splits);
}

// reduce: launch the summing kernel of a split GEMM (false: its consumer
// sums the slices).
int gemm_launch(fg_ctx *ctx, const Planned &P, const char *who, bool reduce = true) {
    if (P.empty) return FG_OK;
    if (P.skinny) {
        fg::gemm::launch_skinny(P.a, P.layout, ctx->stream);
        FG_LAUNCH_CHECK(who);
        return FG_OK;
    }
    switch (P.layout) {
        case FG_NN: fg::gemm::launch_nn(P.a, P.vec, P.pipe, P.ktail, P.cfg, ctx->stream); break;
        case FG_NT:
            fg::gemm::launch_nt(P.a, P.vec, P.pipe, P.ktail, P.cfg, P.pro, ctx->stream);
            break;
        default: fg::gemm::launch_tn(P.a, P.vec, P.pipe, P.ktail, P.cfg, P.pro, ctx->stream); break;
    }
    FG_LAUNCH_CHECK(who);
    if (P.splits > 1 && reduce) {
        launch_reduce(ctx, P.a, P.splits);
        FG_LAUNCH_CHECK(who);
    }
    return FG_OK;
}

int gemm_common(fg_ctx *ctx, int layout, GemmArgs &a, const char *who,
                int pro = fg::gemm::kProNone) {
    Planned P;
    const int rc = gemm_prepare(ctx, layout, a, who, pro, P);
    if (rc) return rc;
    return gemm_launch(ctx, P, who);
}

// The pair kernel that a planned GEMM would take (-1: it does not pair).
int pair_kind(const Planned &P) {
    if (P.empty || P.pro != fg::gemm::kProNone) return -1;
    if (P.skinny) return fg::gemm::kPairSkinny;
    if (!P.vec) return fg::gemm::kPairElem;
    if (P.pipe && !P.ktail && P.cfg == 4) return fg::gemm::kPairPipe;
    if (P.pipe && !P.ktail && P.splits == 1 &&
        ((P.layout == FG_TN && P.cfg == 6) || (P.layout == FG_NT && P.cfg == 7)))
        return fg::gemm::kPairBig;
    if (P.pipe && !P.ktail && P.cfg == 5) return fg::gemm::kPairMid;
    return -1;
}

// Output tiles x and workgroups n of a paired GEMM (sets its tile counts).
void pair_grid(Planned &P, int &x, int &n) {
    if (P.skinny) {
        x = n = fg::gemm::skinny_workgroups(P.a.M);
        return;
    }
    int bm = 64, bn = 64;  // the small pairing kernels' tiles
    if (pair_kind(P) == fg::gemm::kPairBig) {
        bm = 256;
        bn = P.layout == FG_TN ? 256 : 128;
    } else if (pair_kind(P) == fg::gemm::kPairMid) {
        bm = 128;
    }
    P.a.tiles_m = (P.a.M + bm - 1) / bm;
    P.a.tiles_n = (P.a.N + bn - 1) / bn;
    x = P.a.tiles_m * P.a.tiles_n;
    n = x * P.splits;
}

}  // namespace

namespace fg {
int reduce_blocks(const fg_ctx *ctx, int M, int N) {
    const size_t mn = (size_t)M * N;
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    return (int)std::min<size_t>((mn + kThreads - 1) / kThreads, 4 * (size_t)cus);
}

int launch_pending_reduce(fg_ctx *ctx) {
    if (ctx->pending_splits <= 0) return FG_OK;
    GemmArgs a;
    std::memcpy(&a, ctx->pending, sizeof a);
    const int splits = ctx->pending_splits;
    ctx->pending_splits = 0;
    splitk_reduce<<<reduce_blocks(ctx, a.M, a.N), kThreads, 0, ctx->stream>>>(a, splits);
    FG_LAUNCH_CHECK("splitk_reduce");
    return FG_OK;
}

int sgd_step_with_pending(fg_ctx *ctx, fg_mt *mt, float lr, int zero_grad, fg_ctx *held) {
    FG_REQUIRE(ctx && mt && held, FG_ERR_INVALID_ARGUMENT, "sgd_step_with_pending: NULL argument");
    const bool mean = held->mean_dst != nullptr;
    if (held->pending_splits <= 0 && !mean) return fg_sgd_step(ctx, mt, lr, zero_grad);
    FG_HIP(hipSetDevice(ctx->device));
    GemmArgs a{};
    int splits = 1, nred = 0;
    if (held->pending_splits > 0) {
        std::memcpy(&a, held->pending, sizeof a);
        splits = held->pending_splits;
        nred = reduce_blocks(held, a.M, a.N);
        held->pending_splits = 0;
    }
    sgd_and_split_sum<<<mt->nchunks + nred + (mean ? 1 : 0), kThreads, 0, ctx->stream>>>(
        mt->d_tensors, mt->d_chunks, lr, zero_grad, mt->vec, mt->nchunks, a, splits, nred,
        held->mean_src, held->mean_rows, held->mean_dst);
    held->mean_dst = nullptr;
    FG_LAUNCH_CHECK("sgd_and_split_sum");
    return FG_OK;
}

int launch_pending_mean(fg_ctx *ctx) {
    if (!ctx->mean_dst) return FG_OK;
    mean_rows_kernel<<<1, kThreads, 0, ctx->stream>>>(ctx->mean_src, ctx->mean_rows,
                                                      ctx->mean_dst);
    ctx->mean_dst = nullptr;
    FG_LAUNCH_CHECK("mean_rows_kernel");
    return FG_OK;
}

void pending_reduce_ranges(const fg_ctx *ctx, ByteRange out[3]) {
    GemmArgs a;
    std::memcpy(&a, ctx->pending, sizeof a);
    const uintptr_t rows = a.M > 0 ? (uintptr_t)(a.M - 1) : 0;
    out[0] = {(uintptr_t)a.C, (uintptr_t)(a.C + rows * a.ldc + a.N)};
    out[1] = a.mode == 1 && a.act != FG_ACT_NONE && a.Zs
                 ? ByteRange{(uintptr_t)a.Zs, (uintptr_t)(a.Zs + rows * a.ldzs + a.N)}
                 : ByteRange{0, 0};
    out[2] = a.mode == 0 && a.bias ? ByteRange{(uintptr_t)a.bias, (uintptr_t)(a.bias + a.N)}
                                   : ByteRange{0, 0};
}

int gemm_f32_dispatches(fg_ctx *ctx, int layout, int M, int N, int K, const void *A, int lda,
                        const void *B, int ldb, bool colsum) {
    if (!ctx || M <= 0 || N <= 0) return 1;  // no workspace (or nothing to do): no split
    GemmArgs a{};
    a.A = static_cast<const float *>(A);
    a.B = static_cast<const float *>(B);
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.colsum = colsum ? reinterpret_cast<float *>(1) : nullptr;  // only tested for null
    if (K == 0) a.A = a.B;
    bool skinny, vec, pipe, ktail;
    int cfg, splits;
    plan_gemm(ctx, layout, a, skinny, vec, pipe, ktail, cfg, splits);
    return splits > 1 ? 2 : 1;
}
}  // namespace fg

FG_API int fg_gemm_f32(fg_ctx *ctx, int layout, int M, int N, int K, const float *d_A, int lda,
                       const float *d_B, int ldb, const float *d_bias, int act, float *d_C,
                       int ldc, float *d_Z, int ldz, int accumulate) {
    GemmArgs a{};
    a.A = d_A;
    a.B = d_B;
    a.C = d_C;
    a.Z = d_Z;
    a.bias = d_bias;
    a.Zs = nullptr;
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.ldz = d_Z ? ldz : 0;
    a.ldzs = 0;
    a.act = act;
    a.mode = 0;
    a.accumulate = accumulate ? 1 : 0;
    FG_REQUIRE(!d_Z || ldz >= N, FG_ERR_SHAPE, "fg_gemm_f32: ldz=%d < N=%d", ldz, N);
    FG_REQUIRE(!(accumulate && act != FG_ACT_NONE), FG_ERR_INVALID_ARGUMENT,
               "fg_gemm_f32: accumulate requires act NONE");
    return gemm_common(ctx, layout, a, "fg_gemm_f32");
}

FG_API int fg_gemm_bwd_f32(fg_ctx *ctx, int layout, int M, int N, int K, const float *d_A, int lda,
                           const float *d_B, int ldb, int act, const float *d_Zs, int ldzs,
                           float *d_C, int ldc, int accumulate) {
    GemmArgs a{};
    a.A = d_A;
    a.B = d_B;
    a.C = d_C;
    a.Z = nullptr;
    a.bias = nullptr;
    a.Zs = d_Zs;
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.ldz = 0;
    a.ldzs = ldzs;
    a.act = act;
    a.mode = 1;
    a.accumulate = accumulate ? 1 : 0;
    FG_REQUIRE(act == FG_ACT_NONE || (d_Zs && ldzs >= N), FG_ERR_INVALID_ARGUMENT,
               "fg_gemm_bwd_f32: act %d needs Zs with ldzs >= N", act);
    return gemm_common(ctx, layout, a, "fg_gemm_bwd_f32");
}

namespace {
// C (=|+=) A^T.B with colsum (=|+=) the column sums of B (TN); with a
// prologue, B is scaled by act'(Pz) on load and the sums are of the scaled B.
int gemm_dw(fg_ctx *ctx, int M, int N, int K, const float *d_A, int lda, const float *d_B,
            int ldb, float *d_C, int ldc, int accumulate, float *d_colsum, int colsum_accumulate,
            const float *d_Pz, int ldp, int pro, const char *who) {
    GemmArgs a{};
    a.A = d_A;
    a.B = d_B;
    a.C = d_C;
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.act = FG_ACT_NONE;
    a.mode = 0;
    a.accumulate = accumulate ? 1 : 0;
    a.colsum = d_colsum;
    a.colsum_accumulate = colsum_accumulate ? 1 : 0;
    a.Pz = d_Pz;
    a.ldp = ldp;
    if (d_colsum && (M == 0 || K == 0)) {
        // No tile runs the column sums: an empty reduction.
        FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "%s: ctx is NULL", who);
        if (N > 0 && !colsum_accumulate) {  // a fill kernel: safe under stream capture
            const int rc = fg_fill_u32(ctx, d_colsum, 0u, (uint64_t)N);
            if (rc) return rc;
        }
        if (M == 0) return FG_OK;
        a.colsum = nullptr;
    }
    return gemm_common(ctx, FG_TN, a, who, pro);
}
}  // namespace

FG_API int fg_gemm_dw_f32(fg_ctx *ctx, int M, int N, int K, const float *d_A, int lda,
                          const float *d_B, int ldb, float *d_C, int ldc, int accumulate,
                          float *d_colsum, int colsum_accumulate) {
    return gemm_dw(ctx, M, N, K, d_A, lda, d_B, ldb, d_C, ldc, accumulate, d_colsum,
                   colsum_accumulate, nullptr, 0, fg::gemm::kProNone, "fg_gemm_dw_f32");
}

namespace {
// The arguments of the pair's two GEMMs as the single-GEMM entry points build
// them: dW (TN) with the column sums, dX (NT) with act'(Zs).
GemmArgs dw_args(int M, int N, int K, const float *A, int lda, const float *B, int ldb, float *C,
                 int ldc, int accumulate, float *colsum, int colsum_accumulate) {
    GemmArgs a{};
    a.A = A;
    a.B = B;
    a.C = C;
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.act = FG_ACT_NONE;
    a.mode = 0;
    a.accumulate = accumulate ? 1 : 0;
    a.colsum = colsum;
    a.colsum_accumulate = colsum_accumulate ? 1 : 0;
    return a;
}
GemmArgs dx_args(int M, int N, int K, const float *A, int lda, const float *B, int ldb, int act,
                 const float *Zs, int ldzs, float *C, int ldc, int accumulate) {
    GemmArgs a{};
    a.A = A;
    a.B = B;
    a.C = C;
    a.Zs = Zs;
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
    return a;
}

// Both pairable: at most one of them splits K (the slices of a split GEMM
// take the whole workspace), and a kind that pairs only with itself has its
// own kind beside it.
bool pairable(const Planned &P1, const Planned &P2) {
    const int k1 = pair_kind(P1), k2 = pair_kind(P2);
    if (k1 < 0 || k2 < 0 || (P1.splits > 1 && P2.splits > 1)) return false;
    return fg::gemm::pair_exclusive(k1) || fg::gemm::pair_exclusive(k2) ? k1 == k2 : true;
}

// Both validated and planned, and pairable.
bool plan_pair(fg_ctx *ctx, const GemmArgs &w, const GemmArgs &x, Planned &P1, Planned &P2) {
    if (gemm_prepare(ctx, FG_TN, w, "fg_gemm_dw_f32", fg::gemm::kProNone, P1) ||
        gemm_prepare(ctx, FG_NT, x, "fg_gemm_bwd_f32", fg::gemm::kProNone, P2))
        return false;
    return pairable(P1, P2);
}

// Forward GEMM arguments (as fg_gemm_f32 takes them).
GemmArgs fwd_args(int M, int N, int K, const float *A, int lda, const float *B, int ldb,
                  const float *bias, int act, float *C, int ldc, float *Z, int ldz,
                  int accumulate) {
    GemmArgs a{};
    a.A = A;
    a.B = B;
    a.C = C;
    a.Z = Z;
    a.bias = bias;
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.ldz = Z ? ldz : 0;
    a.act = act;
    a.mode = 0;
    a.accumulate = accumulate ? 1 : 0;
    return a;
}

// GEMM 1's slices summed by GEMM 2's skinny kernel: GEMM 1 splits K into at
// most kSkPreMaxSlices slices, without accumulation, its output (N a
// multiple of 4, 16-byte rows) is exactly GEMM 2's A operand, and GEMM 2
// takes the skinny kernel in the NN layout.
bool chainable(const Planned &P1, const Planned &P2) {
    const GemmArgs &a = P1.a, &b = P2.a;
    return !P1.empty && !P2.empty && P1.layout == FG_NN && P2.layout == FG_NN &&
           P1.pro == fg::gemm::kProNone && P1.splits > 1 &&
           P1.splits <= fg::gemm::kSkPreMaxSlices && !a.accumulate && a.mode == 0 &&
           a.N % 4 == 0 && a.vec_out && P2.skinny && b.A == a.C && b.lda == a.ldc &&
           b.K == a.N && b.M == a.M;
}

// The kernel choices alone, for counting dispatches: no validation, no error
// message, operands not bound yet taken as 16-byte aligned.
void plan_quiet(fg_ctx *ctx, int layout, const GemmArgs &a0, Planned &P) {
    P.a = a0;
    P.layout = layout;
    const float *aligned = reinterpret_cast<const float *>(256);
    if (!P.a.A) P.a.A = aligned;
    if (!P.a.B) P.a.B = aligned;
    plan_gemm(ctx, layout, P.a, P.skinny, P.vec, P.pipe, P.ktail, P.cfg, P.splits);
}
}  // namespace

namespace fg {
// A layer's weight gradient dW (=|+=) X^T.dZ with dbias (=|+=) the column
// sums of dZ (as fg_gemm_dw_f32) and its data gradient dX (=|+=)
// (dZ.W^T) * act'(Zs) (as fg_gemm_bwd_f32, NT): independent GEMMs, one
// launch when both take small 256-thread kernels, else one after the other.
// The same results, bit for bit, either way.
int gemm_dw_dx_f32(fg_ctx *ctx, int M1, int N1, int K1, const float *A1, int lda1,
                   const float *B1, int ldb1, float *C1, int ldc1, int acc1, float *colsum,
                   int colsum_acc, int M2, int N2, int K2, const float *A2, int lda2,
                   const float *B2, int ldb2, int act, const float *Zs, int ldzs, float *C2,
                   int ldc2, int acc2) {
    auto separate = [&]() {
        const int rc = fg_gemm_dw_f32(ctx, M1, N1, K1, A1, lda1, B1, ldb1, C1, ldc1, acc1, colsum,
                                      colsum_acc);
        if (rc) return rc;
        return fg_gemm_bwd_f32(ctx, FG_NT, M2, N2, K2, A2, lda2, B2, ldb2, act, Zs, ldzs, C2, ldc2,
                               acc2);
    };
    // Empty shapes (the column-sum fill of an empty reduction) stay separate.
    if (!ctx || M1 <= 0 || N1 <= 0 || K1 <= 0 || M2 <= 0 || N2 <= 0 || K2 <= 0) return separate();
    FG_REQUIRE(act == FG_ACT_NONE || (Zs && ldzs >= N2), FG_ERR_INVALID_ARGUMENT,
               "fg_gemm_bwd_f32: act %d needs Zs with ldzs >= N", act);
    Planned P1, P2;
    if (!plan_pair(ctx, dw_args(M1, N1, K1, A1, lda1, B1, ldb1, C1, ldc1, acc1, colsum, colsum_acc),
                   dx_args(M2, N2, K2, A2, lda2, B2, ldb2, act, Zs, ldzs, C2, ldc2, acc2), P1, P2))
        return separate();
    int x1, n1, x2, n2;
    pair_grid(P1, x1, n1);
    pair_grid(P2, x2, n2);
    fg::gemm::launch_pair(pair_kind(P1), pair_kind(P2), P1.a, P2.a, x1, n1, x2, n2, ctx->stream);
    FG_LAUNCH_CHECK("gemm_dw_dx_f32");
    for (const Planned *P : {&P1, &P2})
        if (P->splits > 1) {
            launch_reduce(ctx, P->a, P->splits);
            FG_LAUNCH_CHECK("gemm_dw_dx_f32");
        }
    return FG_OK;
}

// Two forward GEMMs in a row where the second reads the first's output as
// its A operand (NN both; GEMM 1 with bias / activation / Z as fg_gemm_f32):
// when GEMM 1 splits K and GEMM 2 takes the skinny kernel, GEMM 2's kernel
// sums GEMM 1's slices (slice order, GEMM 1's epilogue, GEMM 1's outputs
// written) instead of a summing kernel -- one dispatch fewer, the same bits.
// Otherwise the two calls one after the other.
int gemm_fwd_chain_f32(fg_ctx *ctx, int M1, int N1, int K1, const float *A1, int lda1,
                       const float *B1, int ldb1, const float *bias1, int act1, float *C1,
                       int ldc1, float *Z1, int ldz1, int M2, int N2, int K2, const float *A2,
                       int lda2, const float *B2, int ldb2, const float *bias2, int act2,
                       float *C2, int ldc2, float *Z2, int ldz2, int acc2, const CeOut *ce,
                       bool *ce_done) {
    if (ce_done) *ce_done = false;
    auto separate = [&]() {
        const int rc = fg_gemm_f32(ctx, FG_NN, M1, N1, K1, A1, lda1, B1, ldb1, bias1, act1, C1,
                                   ldc1, Z1, ldz1, 0);
        if (rc) return rc;
        return fg_gemm_f32(ctx, FG_NN, M2, N2, K2, A2, lda2, B2, ldb2, bias2, act2, C2, ldc2, Z2,
                           ldz2, acc2);
    };
    if (!ctx || (Z1 && ldz1 < N1) || (Z2 && ldz2 < N2) || (acc2 && act2 != FG_ACT_NONE))
        return separate();  // the plain calls report the argument errors
    Planned P1, P2;
    if (gemm_prepare(ctx, FG_NN, fwd_args(M1, N1, K1, A1, lda1, B1, ldb1, bias1, act1, C1, ldc1,
                                          Z1, ldz1, 0),
                     "fg_gemm_f32", fg::gemm::kProNone, P1) ||
        gemm_prepare(ctx, FG_NN, fwd_args(M2, N2, K2, A2, lda2, B2, ldb2, bias2, act2, C2, ldc2,
                                          Z2, ldz2, acc2),
                     "fg_gemm_f32", fg::gemm::kProNone, P2) ||
        !chainable(P1, P2)) {
        fg::clear_error();
        return separate();
    }
    // The loss too when its logits are this GEMM's whole output.
    const bool with_ce = ce && ce_done && act2 == FG_ACT_NONE && !acc2 && N2 <= 16 &&
                         M2 <= 1024 && ce->labels && ce->row_loss && ce->dlogits &&
                         ce->ldd >= N2 && (!ce->probs || ce->ldp >= N2);
    if (int rc = gemm_launch(ctx, P1, "gemm_fwd_chain_f32", false)) return rc;
    fg::gemm::launch_skinny_pre(P2.a, P1.a, ctx->stream, with_ce ? ce : nullptr);
    FG_LAUNCH_CHECK("gemm_fwd_chain_f32");
    if (with_ce) *ce_done = true;
    return FG_OK;
}

// Dispatches of gemm_fwd_chain_f32 for these operands (no launch).
int gemm_fwd_chain_dispatches(fg_ctx *ctx, int M1, int N1, int K1, const void *A1, int lda1,
                              const void *B1, int ldb1, const void *bias1, void *C1, int ldc1,
                              void *Z1, int ldz1, int M2, int N2, int K2, const void *A2, int lda2,
                              const void *B2, int ldb2) {
    const int sep = gemm_f32_dispatches(ctx, FG_NN, M1, N1, K1, A1, lda1, B1, ldb1, false) +
                    gemm_f32_dispatches(ctx, FG_NN, M2, N2, K2, A2, lda2, B2, ldb2, false);
    if (!ctx || M1 <= 0 || N1 <= 0 || M2 <= 0 || N2 <= 0) return sep;
    Planned P1, P2;
    GemmArgs a1 = fwd_args(M1, N1, K1, (const float *)A1, lda1, (const float *)B1, ldb1,
                           (const float *)bias1, FG_ACT_NONE, (float *)C1, ldc1, (float *)Z1,
                           ldz1, 0);
    plan_quiet(ctx, FG_NN, a1, P1);
    plan_quiet(ctx, FG_NN, fwd_args(M2, N2, K2, (const float *)A2, lda2, (const float *)B2, ldb2,
                                    nullptr, FG_ACT_NONE, nullptr, N2, nullptr, 0, 0), P2);
    return chainable(P1, P2) ? 2 : sep;
}

// A small head's weight gradient (with its bias gradient; TN) beside a
// layer's dW and dX (as gemm_dw_dx_f32): one launch when the head's takes
// the skinny kernel and the two pair with 256-thread kernels; otherwise the
// head's alone, then the pair.  The same bits either way.
int gemm_dw_dw_dx_f32(fg_ctx *ctx, int M0, int N0, int K0, const float *A0, int lda0,
                      const float *B0, int ldb0, float *C0, int ldc0, int acc0, float *colsum0,
                      int colsum_acc0, int M1, int N1, int K1, const float *A1, int lda1,
                      const float *B1, int ldb1, float *C1, int ldc1, int acc1, float *colsum1,
                      int colsum_acc1, int M2, int N2, int K2, const float *A2, int lda2,
                      const float *B2, int ldb2, int act, const float *Zs, int ldzs, float *C2,
                      int ldc2, int acc2) {
    auto separate = [&]() {
        const int rc = fg_gemm_dw_f32(ctx, M0, N0, K0, A0, lda0, B0, ldb0, C0, ldc0, acc0, colsum0,
                                      colsum_acc0);
        if (rc) return rc;
        return gemm_dw_dx_f32(ctx, M1, N1, K1, A1, lda1, B1, ldb1, C1, ldc1, acc1, colsum1,
                              colsum_acc1, M2, N2, K2, A2, lda2, B2, ldb2, act, Zs, ldzs, C2, ldc2,
                              acc2);
    };
    if (!ctx || M0 <= 0 || N0 <= 0 || K0 <= 0 || M1 <= 0 || N1 <= 0 || K1 <= 0 || M2 <= 0 ||
        N2 <= 0 || K2 <= 0 || (act != FG_ACT_NONE && (!Zs || ldzs < N2)))
        return separate();
    Planned P0, P1, P2;
    if (gemm_prepare(ctx, FG_TN, dw_args(M0, N0, K0, A0, lda0, B0, ldb0, C0, ldc0, acc0, colsum0,
                                         colsum_acc0),
                     "fg_gemm_dw_f32", fg::gemm::kProNone, P0) ||
        !plan_pair(ctx, dw_args(M1, N1, K1, A1, lda1, B1, ldb1, C1, ldc1, acc1, colsum1, colsum_acc1),
                   dx_args(M2, N2, K2, A2, lda2, B2, ldb2, act, Zs, ldzs, C2, ldc2, acc2), P1, P2) ||
        pair_kind(P0) != fg::gemm::kPairSkinny || fg::gemm::pair_exclusive(pair_kind(P1))) {
        fg::clear_error();
        return separate();
    }
    int x0, n0, x1, n1, x2, n2;
    pair_grid(P0, x0, n0);
    pair_grid(P1, x1, n1);
    pair_grid(P2, x2, n2);
    fg::gemm::launch_triple(P0.a, n0, pair_kind(P1), P1.a, x1, n1, pair_kind(P2), P2.a, x2, n2,
                            ctx->stream);
    FG_LAUNCH_CHECK("gemm_dw_dw_dx_f32");
    for (const Planned *P : {&P1, &P2})
        if (P->splits > 1) {
            launch_reduce(ctx, P->a, P->splits);
            FG_LAUNCH_CHECK("gemm_dw_dw_dx_f32");
        }
    return FG_OK;
}

int gemm_skinny_max_n() { return fg::gemm::kSkinnyN; }

// Dispatches of gemm_dw_dw_dx_f32 for these shapes (no launch).
int gemm_dw_dw_dx_dispatches(fg_ctx *ctx, int M0, int N0, int K0, const void *A0, int lda0,
                             const void *B0, int ldb0, int M1, int N1, int K1, const void *A1,
                             int lda1, const void *B1, int ldb1, int M2, int N2, int K2,
                             const void *A2, int lda2, const void *B2, int ldb2) {
    const int sep = gemm_f32_dispatches(ctx, FG_TN, M0, N0, K0, A0, lda0, B0, ldb0, true) +
                    gemm_dw_dx_dispatches(ctx, M1, N1, K1, A1, lda1, B1, ldb1, M2, N2, K2, A2,
                                          lda2, B2, ldb2);
    if (!ctx || M0 <= 0 || N0 <= 0 || K0 <= 0 || M1 <= 0 || N1 <= 0 || K1 <= 0 || M2 <= 0 ||
        N2 <= 0 || K2 <= 0)
        return sep;
    float *c = reinterpret_cast<float *>(256);
    Planned P0, P1, P2;
    plan_quiet(ctx, FG_TN, dw_args(M0, N0, K0, (const float *)A0, lda0, (const float *)B0, ldb0,
                                   c, N0, 0, c, 0), P0);
    plan_quiet(ctx, FG_TN, dw_args(M1, N1, K1, (const float *)A1, lda1, (const float *)B1, ldb1,
                                   c, N1, 0, c, 0), P1);
    plan_quiet(ctx, FG_NT, dx_args(M2, N2, K2, (const float *)A2, lda2, (const float *)B2, ldb2,
                                   FG_ACT_NONE, nullptr, 0, c, N2, 0), P2);
    if (pair_kind(P0) != fg::gemm::kPairSkinny || !pairable(P1, P2) ||
        fg::gemm::pair_exclusive(pair_kind(P1)))
        return sep;
    return 1 + (P1.splits > 1) + (P2.splits > 1);
}

// Dispatches of gemm_dw_dx_f32 for these shapes: 1 (+1 per split GEMM) when
// the two pair, else the sum of the two calls'.  No launch.
int gemm_dw_dx_dispatches(fg_ctx *ctx, int M1, int N1, int K1, const void *A1, int lda1,
                          const void *B1, int ldb1, int M2, int N2, int K2, const void *A2,
                          int lda2, const void *B2, int ldb2) {
    const int sep = gemm_f32_dispatches(ctx, FG_TN, M1, N1, K1, A1, lda1, B1, ldb1, true) +
                    gemm_f32_dispatches(ctx, FG_NT, M2, N2, K2, A2, lda2, B2, ldb2, false);
    if (!ctx || M1 <= 0 || N1 <= 0 || K1 <= 0 || M2 <= 0 || N2 <= 0 || K2 <= 0) return sep;
    // Dummy aligned outputs: only the operands' alignment enters the choice.
    float *c = reinterpret_cast<float *>(256);
    Planned P1, P2;
    plan_quiet(ctx, FG_TN, dw_args(M1, N1, K1, (const float *)A1, lda1, (const float *)B1, ldb1,
                                   c, N1, 0, c, 0), P1);
    plan_quiet(ctx, FG_NT, dx_args(M2, N2, K2, (const float *)A2, lda2, (const float *)B2, ldb2,
                                   FG_ACT_NONE, nullptr, 0, c, N2, 0), P2);
    if (!pairable(P1, P2)) return sep;
    return 1 + (P1.splits > 1) + (P2.splits > 1);
}
}  // namespace fg

FG_API int fg_linear_bwd_f32(fg_ctx *ctx, int act, int M, int N, int K, const float *d_X,
                             int ldx, const float *d_W, int ldw, const float *d_Zs, int ldzs,
                             const float *d_dC, int lddc, float *d_dX, int lddx, float *d_dW,
                             int lddw, float *d_dbias, int accumulate, float *d_dZ, int lddz) {
    const char *who = "fg_linear_bwd_f32";
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "%s: ctx is NULL", who);
    FG_REQUIRE(act >= FG_ACT_NONE && act <= FG_ACT_GELU, FG_ERR_INVALID_ARGUMENT,
               "%s: bad act %d", who, act);
    FG_REQUIRE(M >= 0 && N >= 0 && K >= 0, FG_ERR_SHAPE, "%s: negative dimension", who);
    if (N == 0) return FG_OK;
    FG_REQUIRE(d_dC && lddc >= N, FG_ERR_INVALID_ARGUMENT, "%s: dC NULL or lddc < N", who);
    FG_REQUIRE(act == FG_ACT_NONE || (d_Zs && ldzs >= N), FG_ERR_INVALID_ARGUMENT,
               "%s: act %d needs Zs with ldzs >= N", who, act);
    FG_REQUIRE(!d_dZ || lddz >= N, FG_ERR_INVALID_ARGUMENT, "%s: lddz < N", who);
    const bool want_w = d_dW && K > 0;
    if (want_w)
        FG_REQUIRE(d_X && ldx >= K && lddw >= N, FG_ERR_INVALID_ARGUMENT,
                   "%s: X NULL or ldx < K or lddw < N", who);
    const bool want_x = d_dX && K > 0;
    if (want_x)
        FG_REQUIRE(d_W && ldw >= N && lddx >= K, FG_ERR_INVALID_ARGUMENT,
                   "%s: W NULL or ldw < N or lddx < K", who);
    using namespace fg::gemm;
    // The GEMMs' dC operand: dC itself with the prologue, or the materialised
    // dZ (act NONE: dC is dZ).
    const float *g = d_dC;
    int ldg = lddc, pro_tn = kProNone, pro_nt = kProNone;
    bool dbias_done = false;
    if (act != FG_ACT_NONE && d_dZ) {
        // One pass over dC and Zs writes dZ and, when asked, sums its columns.
        FG_HIP(hipSetDevice(ctx->device));
        const fg::colsum::Split sp =
            fg::colsum::split_of(ctx->cu_count > 0 ? ctx->cu_count : 256, M, N);
        float *partial = (float *)fg::workspace(
            ctx, std::max<uint64_t>(sp.partial_floats(N), 1) * sizeof(float));
        if (!partial) return FG_ERR_OUT_OF_MEMORY;
        FG_HIP(fg::colsum::launch(ctx->stream, sp, FG_DTYPE_F32, M, N, d_dC, lddc, d_dbias,
                                  accumulate, partial, act, d_Zs, ldzs, d_dZ, lddz));
        dbias_done = true;
        g = d_dZ;
        ldg = lddz;
    } else if (act != FG_ACT_NONE) {
        pro_tn = act == FG_ACT_RELU ? kProBReLU : kProBGelu;
        pro_nt = act == FG_ACT_RELU ? kProAReLU : kProAGelu;
    }
    if (want_w) {  // dW = X^T.dZ (TN, dZ the B operand), dbias from its tiles if still due
        const int rc = gemm_dw(ctx, K, N, M, d_X, ldx, g, ldg, d_dW, lddw, accumulate,
                               dbias_done ? nullptr : d_dbias, accumulate, d_Zs, ldzs, pro_tn,
                               who);
        if (rc) return rc;
    } else if (d_dbias && !dbias_done) {  // dbias alone: the column reduction (+ prologue)
        FG_HIP(hipSetDevice(ctx->device));
        const fg::colsum::Split sp =
            fg::colsum::split_of(ctx->cu_count > 0 ? ctx->cu_count : 256, M, N);
        float *partial = (float *)fg::workspace(
            ctx, std::max<uint64_t>(sp.partial_floats(N), 1) * sizeof(float));
        if (!partial) return FG_ERR_OUT_OF_MEMORY;
        FG_HIP(fg::colsum::launch(ctx->stream, sp, FG_DTYPE_F32, M, N, d_dC, lddc, d_dbias,
                                  accumulate, partial, act, d_Zs, ldzs));
    }
    if (want_x) {  // dX = dZ.W^T (NT, dZ the A operand)
        GemmArgs a{};
        a.A = g;
        a.lda = ldg;
        a.B = d_W;
        a.ldb = ldw;
        a.C = d_dX;
        a.ldc = lddx;
        a.M = M;
        a.N = K;
        a.K = N;
        a.mode = 1;
        a.act = FG_ACT_NONE;
        a.accumulate = accumulate ? 1 : 0;
        a.Pz = d_Zs;
        a.ldp = ldzs;
        const int rc = gemm_common(ctx, FG_NT, a, who, pro_nt);
        if (rc) return rc;
    }
    return FG_OK;
}

FG_API int fg_matmul_bwd_f32(fg_ctx *ctx, int M, int N, int K, const float *d_X, int ldx,
                             const float *d_W, int ldw, const float *d_dZ, int lddz, int act,
                             const float *d_Zs, int ldzs, float *d_dX, int lddx, float *d_dW,
                             int lddw, float *d_dbias, int accumulate) {
    const char *who = "fg_matmul_bwd_f32";
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
    return fg::gemm_dw_dx_f32(ctx, K, N, M, d_X, ldx, d_dZ, lddz, d_dW, lddw, accumulate,
                              d_dbias, accumulate, M, K, N, d_dZ, lddz, d_W, ldw, act, d_Zs,
                              ldzs, d_dX, lddx, accumulate);
}

namespace fg {
uint64_t bias_grad_ws_bytes(int cus, int M, int N) {
    return colsum::split_of(cus > 0 ? cus : 256, M, N).partial_floats(N) * sizeof(float);
}
}  // namespace fg

FG_API int fg_bias_grad(fg_ctx *ctx, int dtype, int M, int N, const void *d_dZ, int ld,
                        void *d_dbias, int accumulate) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "fg_bias_grad: ctx is NULL");
    FG_REQUIRE(dtype >= FG_DTYPE_F32 && dtype <= FG_DTYPE_BF16, FG_ERR_INVALID_ARGUMENT,
               "fg_bias_grad: bad dtype %d", dtype);
    FG_REQUIRE(M >= 0 && N >= 0 && ld >= N, FG_ERR_SHAPE,
               "fg_bias_grad: bad shape M=%d N=%d ld=%d", M, N, ld);
    if (N == 0) return FG_OK;
    FG_REQUIRE(d_dZ && d_dbias, FG_ERR_INVALID_ARGUMENT, "fg_bias_grad: NULL pointer");
    FG_HIP(hipSetDevice(ctx->device));
    const fg::colsum::Split sp =
        fg::colsum::split_of(ctx->cu_count > 0 ? ctx->cu_count : 256, M, N);
    float *partial = (float *)fg::workspace(ctx, std::max<uint64_t>(sp.partial_floats(N), 1) *
                                                     sizeof(float));
    if (!partial) return FG_ERR_OUT_OF_MEMORY;
    FG_HIP(fg::colsum::launch(ctx->stream, sp, dtype, M, N, d_dZ, ld, d_dbias, accumulate,
                              partial));
    return FG_OK;
}

FG_API int fg_bias_grad_f32(fg_ctx *ctx, int M, int N, const float *d_dZ, int ld, float *d_dbias,
                            int accumulate) {
    return fg_bias_grad(ctx, FG_DTYPE_F32, M, N, d_dZ, ld, d_dbias, accumulate);
}
