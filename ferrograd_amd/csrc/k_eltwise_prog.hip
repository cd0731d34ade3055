// k_eltwise_prog.hip -- the elementwise-program kernel (see fg_eltwise.h).
// Every lane runs the same instruction stream (uniform branches), so the
// interpretation costs scalar-unit work only; the kernel stays HBM-bound
// for the short programs the planner emits.
#include <hip/hip_runtime.h>

#include "fg_act.h"
#include "fg_eltwise.h"
#include "fg_half.h"
#include "fg_internal.h"

namespace fg {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float elt_load(const EltProgram &p, int s, int mode, int dt,
                                          uint64_t i) {
    const uint64_t j = mode == kModeScalar ? 0 : mode == kModeRow ? i % p.cols : i;
    return load_as_f(p.src[s], dt, j);
}

__global__ __launch_bounds__(kThreads) void eltwise_prog_kernel(const EltProgram p) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < p.n; i += stride) {
        float r[kEltRegs];
#pragma unroll
        for (int k = 0; k < kEltRegs; ++k) r[k] = 0.0f;
        for (int k = 0; k < p.n_instr; ++k) {
            const EltInstr in = p.ins[k];
            switch (in.op) {
                case kEltLoad: r[in.dst & 15] = elt_load(p, in.a, in.c, in.b, i); break;
                case kEltImm: r[in.dst & 15] = in.imm; break;
                case kEltStore: store_from_f(p.dst[in.a], in.c, i, r[in.b & 15]); break;
                case kEltAccum:
                    store_from_f(p.dst[in.a], in.c, i,
                                 load_as_f(p.dst[in.a], in.c, i) + r[in.b & 15]);
                    break;
                case kEltRound: r[in.dst & 15] = round_to(in.c, r[in.a & 15]); break;
                case kEltAdd: r[in.dst & 15] = r[in.a & 15] + r[in.b & 15]; break;
                case kEltSub: r[in.dst & 15] = r[in.a & 15] - r[in.b & 15]; break;
                case kEltMul: r[in.dst & 15] = r[in.a & 15] * r[in.b & 15]; break;
                case kEltDiv: r[in.dst & 15] = r[in.a & 15] / r[in.b & 15]; break;
                case kEltNeg: r[in.dst & 15] = -r[in.a & 15]; break;
                case kEltRelu: r[in.dst & 15] = act_fwd(kActRelu, r[in.a & 15]); break;
                case kEltGelu: r[in.dst & 15] = act_fwd(kActGelu, r[in.a & 15]); break;
                case kEltElu: {
                    const float x = r[in.a & 15];
                    r[in.dst & 15] = x >= 0.0f ? x : expf(x) - 1.0f;
                    break;
                }
                case kEltTanh: r[in.dst & 15] = tanhf(r[in.a & 15]); break;
                case kEltExp: r[in.dst & 15] = expf(r[in.a & 15]); break;
                case kEltLog: r[in.dst & 15] = logf(r[in.a & 15]); break;
                case kEltAbs: r[in.dst & 15] = fabsf(r[in.a & 15]); break;
                case kEltReluD: r[in.dst & 15] = act_grad(kActRelu, r[in.a & 15]); break;
                case kEltGeluD: r[in.dst & 15] = act_grad(kActGelu, r[in.a & 15]); break;
                case kEltEluD: {
                    const float x = r[in.a & 15];
                    r[in.dst & 15] = x >= 0.0f ? 1.0f : expf(x);
                    break;
                }
                case kEltSign: {
                    const float x = r[in.a & 15];
                    r[in.dst & 15] = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
                    break;
                }
                case kEltLabelEq: {
                    const uint64_t row = i / p.cols, col = i % p.cols;
                    r[in.dst & 15] = (p.labels[row] == (uint32_t)col) ? 1.0f : 0.0f;
                    break;
                }
                case kEltSelect:
                    r[in.dst & 15] = r[in.a & 15] != 0.0f ? r[in.b & 15] : r[in.c & 15];
                    break;
                case kEltMax: r[in.dst & 15] = fmaxf(r[in.a & 15], r[in.b & 15]); break;
                default: break;
            }
        }
    }
}

}  // namespace

// Validates the program's indices on the host (so the kernel never reads a
// source or writes a destination that was not supplied) and launches it.
int launch_eltwise(fg_ctx *ctx, const EltProgram &p) {
    if (p.n == 0) return FG_OK;
    FG_REQUIRE(p.n_instr >= 0 && p.n_instr <= kEltMaxInstr, FG_ERR_INTERNAL,
               "eltwise program: %d instructions (max %d)", p.n_instr, kEltMaxInstr);
    bool needs_cols = false;
    for (int k = 0; k < p.n_instr; ++k) {
        const EltInstr &in = p.ins[k];
        if (in.op == kEltLoad) {
            FG_REQUIRE(in.a < kEltMaxSrc && p.src[in.a], FG_ERR_INTERNAL,
                       "eltwise program: load of missing source %d", in.a);
            FG_REQUIRE(in.c <= kModeScalar, FG_ERR_INTERNAL,
                       "eltwise program: bad addressing mode %d", in.c);
            FG_REQUIRE(in.b <= kBF16, FG_ERR_INTERNAL, "eltwise program: bad load type %d",
                       in.b);
            if (in.c == kModeRow) needs_cols = true;
        }
        if (in.op == kEltStore || in.op == kEltAccum) {
            FG_REQUIRE(in.a < kEltMaxDst && p.dst[in.a], FG_ERR_INTERNAL,
                       "eltwise program: store to missing destination %d", in.a);
            FG_REQUIRE(in.c <= kBF16, FG_ERR_INTERNAL, "eltwise program: bad store type %d",
                       in.c);
        }
        if (in.op == kEltRound)
            FG_REQUIRE(in.c <= kBF16, FG_ERR_INTERNAL, "eltwise program: bad round type %d",
                       in.c);
        if (in.op == kEltLabelEq) {
            FG_REQUIRE(p.labels, FG_ERR_INTERNAL, "eltwise program: labels missing");
            needs_cols = true;
        }
    }
    FG_REQUIRE(!needs_cols || p.cols > 0, FG_ERR_INTERNAL, "eltwise program: cols is 0");
    uint64_t blocks = (p.n + kThreads - 1) / kThreads;
    const uint64_t cap = (uint64_t)(ctx->cu_count > 0 ? ctx->cu_count : 256) * 8;
    if (blocks > cap) blocks = cap;
    eltwise_prog_kernel<<<(unsigned)blocks, kThreads, 0, ctx->stream>>>(p);
    FG_LAUNCH_CHECK("eltwise_prog_kernel");
    return FG_OK;
}

}  // namespace fg
