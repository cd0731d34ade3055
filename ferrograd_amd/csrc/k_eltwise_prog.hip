// k_eltwise_prog.hip -- the elementwise-program kernel (see fg_eltwise.h).
// Every lane runs the same instruction stream (uniform branches), so the
// interpretation costs scalar-unit work only; the kernel stays HBM-bound
// for the short programs the planner emits.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "fg_elt_ops.h"
#include "fg_eltwise.h"
#include "fg_half.h"
#include "fg_internal.h"

namespace fg {

namespace {

constexpr int kThreads = 256;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Each thread runs the program over a quad of 4 consecutive elements
// (i0 .. i0+3, i0 % 4 == 0): registers are f32x4, and a load or store moves
// the quad with one 16-byte (fp32) or 8-byte (16-bit) access when the
// pointer allows it (the pointer test is uniform, so it costs scalar work).
// Quads that cross the end of the tensor, unaligned pointers and the
// row-broadcast of a row whose length is not a multiple of 4 go element by
// element.  Every element sees the same fp32 operations as the one-element
// form, in the same order: the results are bit-identical.
__device__ __forceinline__ bool quad_aligned(const void *q, int dt) {
    return (((uintptr_t)q) & (dt == kF32 ? 15u : 7u)) == 0;
}

// NT: streaming (non-temporal) loads and stores, for tensors far larger than
// the caches (the copy-like streams of such programs ran 6 % faster).
template <bool NT>
__device__ __forceinline__ f32x4 quad_get(const void *q, int dt, uint64_t j) {
    if (dt == kF32) {
        const f32x4 *a = reinterpret_cast<const f32x4 *>(static_cast<const float *>(q) + j);
        return NT ? __builtin_nontemporal_load(a) : *a;
    }
    const u32x2 *a = reinterpret_cast<const u32x2 *>(static_cast<const uint16_t *>(q) + j);
    const u32x2 w = NT ? __builtin_nontemporal_load(a) : *a;
    return f32x4{h16_to_f(dt, (uint16_t)(w.x & 0xffffu)), h16_to_f(dt, (uint16_t)(w.x >> 16)),
                 h16_to_f(dt, (uint16_t)(w.y & 0xffffu)), h16_to_f(dt, (uint16_t)(w.y >> 16))};
}

template <bool NT>
__device__ __forceinline__ void quad_put(void *q, int dt, uint64_t j, f32x4 v) {
    if (dt == kF32) {
        f32x4 *a = reinterpret_cast<f32x4 *>(static_cast<float *>(q) + j);
        if (NT)
            __builtin_nontemporal_store(v, a);
        else
            *a = v;
        return;
    }
    u32x2 w;
    w.x = (uint32_t)f_to_h16(dt, v[0]) | ((uint32_t)f_to_h16(dt, v[1]) << 16);
    w.y = (uint32_t)f_to_h16(dt, v[2]) | ((uint32_t)f_to_h16(dt, v[3]) << 16);
    u32x2 *a = reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(q) + j);
    if (NT)
        __builtin_nontemporal_store(w, a);
    else
        *a = w;
}

// Source s at elements i0 .. i0+nv-1 (missing lanes of a partial quad are 0).
template <bool NT>
__device__ __forceinline__ f32x4 quad_load(const EltProgram &p, int s, int mode, int dt,
                                           uint64_t i0, int nv) {
    const void *q = p.src[s];
    if (mode == kModeScalar) {
        const float x = load_as_f(q, dt, 0);
        return f32x4{x, x, x, x};
    }
    if (mode == kModeFull) {
        if (nv == 4 && quad_aligned(q, dt)) return quad_get<NT>(q, dt, i0);
        f32x4 r{0.f, 0.f, 0.f, 0.f};
        for (int e = 0; e < nv; ++e) r[e] = load_as_f(q, dt, i0 + e);
        return r;
    }
    // Row broadcast: element i reads src[i % cols].
    const uint32_t c0 = (uint32_t)(i0 % p.cols);
    if (nv == 4 && p.cols % 4 == 0 && quad_aligned(q, dt)) return quad_get<false>(q, dt, c0);
    f32x4 r{0.f, 0.f, 0.f, 0.f};
    for (int e = 0; e < nv; ++e) r[e] = load_as_f(q, dt, (c0 + (uint32_t)e) % p.cols);
    return r;
}

template <bool NT>
__device__ __forceinline__ void quad_store(const EltProgram &p, int d, int dt, uint64_t i0, int nv,
                                           f32x4 v, bool accum) {
    void *q = p.dst[d];
    if (nv == 4 && quad_aligned(q, dt)) {
        if (accum) v += quad_get<NT>(q, dt, i0);
        quad_put<NT>(q, dt, i0, v);
        return;
    }
    for (int e = 0; e < nv; ++e)
        store_from_f(q, dt, i0 + e, accum ? load_as_f(q, dt, i0 + e) + v[e] : v[e]);
}

template <class F>
__device__ __forceinline__ f32x4 quad_map(f32x4 x, F f) {
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = f(x[e]);
    return r;
}

// The register file holds R * U <= kEltRegs quads per thread: R program
// registers (a power of two) for each of the U quads the thread runs the
// program over in one pass.  Slot u * R + r holds register r of quad u, in
// four arrays (one per element of a quad) of R * U floats, all indexed by
// the same uniform number: the compiler reads arrays of 12 or more through
// the GPU's relative register addressing (one index setup serves every quad,
// since quad u only adds the constant u * R), and smaller ones through
// select chains.
//
// Every lane runs the same instruction stream, so decoding an instruction,
// branching on its op and reading its pointers is scalar work done once per
// wave and pass; the scalar unit is shared by the CU's waves and bounds
// short programs on one quad per thread.  U quads per pass spread that work
// over 4 * U elements per lane, while the register file and the U quads'
// operands set how many waves fit a SIMD, and with them the bytes in flight:
// launch_eltwise allocates the program's registers by liveness and picks the
// file from a measured sweep.  Thread t of a workgroup takes quads
// base + u * kThreads + t (u < U), so each load and store of a pass stays
// coalesced.  The pass loop is uniform: a lane past the end takes an empty
// quad (loads give 0, stores skip), so the interpreter runs outside any
// divergent region.
template <int R, int U, bool NT>
__global__ __launch_bounds__(kThreads) void eltwise_prog_kernel(const EltProgram p) {
    static_assert(R * U <= kEltRegs && (R & (R - 1)) == 0, "the file holds R x U quads per thread");
    static_assert(kEltPre <= R, "prefetched sources occupy registers 0 .. n_pre-1");
    constexpr int kFile = R * U;
    const uint64_t nq = (p.n + 3) / 4;
    const uint64_t span = (uint64_t)kThreads * U;
    const uint64_t stride = (uint64_t)gridDim.x * span;
    float f0[kFile], f1[kFile], f2[kFile], f3[kFile];
#pragma unroll
    for (int k = 0; k < kFile; ++k) f0[k] = f1[k] = f2[k] = f3[k] = 0.0f;
    // u is a compile-time constant at every call (unrolled loops), r a
    // uniform run-time register number kept inside the file by the mask.
    auto get = [&](int u, int r) {
        const int k = u * R + (r & (R - 1));
        return f32x4{f0[k], f1[k], f2[k], f3[k]};
    };
    auto set = [&](int u, int r, f32x4 v) {
        const int k = u * R + (r & (R - 1));
        f0[k] = v[0];
        f1[k] = v[1];
        f2[k] = v[2];
        f3[k] = v[3];
    };
    for (uint64_t base = (uint64_t)blockIdx.x * span; base < nq; base += stride) {
        uint64_t i0[U];
        int nv[U];  // elements of quad u (0 past the end: loads give 0, stores skip)
        // The prefetched sources, every load issued before the program runs:
        // a value must be present when the program first reads the file (a
        // run-time index), so loads the program issues itself wait in turn.
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t qi = base + (uint64_t)u * kThreads + threadIdx.x;
            i0[u] = 4 * qi;
            nv[u] = qi >= nq ? 0 : (p.n - i0[u] >= 4 ? 4 : (int)(p.n - i0[u]));
#pragma unroll
            for (int j = 0; j < kEltPre; ++j)
                if (j < p.n_pre)
                    set(u, j, quad_load<NT>(p, p.pre_src[j], kModeFull, p.pre_dt[j], i0[u], nv[u]));
        }
        for (int k = 0; k < p.n_instr; ++k) {
            const EltInstr in = p.ins[k];
            // One read site per operand and one write site for the result
            // (each indexed access costs scalar work to set up).
            f32x4 x[U], y[U], o[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                x[u] = get(u, in.a);
                y[u] = get(u, in.b);
                o[u] = x[u];
            }
            bool wr = true;  // the instruction writes register in.dst
            auto unary = [&](auto f) {
#pragma unroll
                for (int u = 0; u < U; ++u) o[u] = quad_map(x[u], f);
            };
            switch (in.op) {
                case kEltLoad:
#pragma unroll
                    for (int u = 0; u < U; ++u) o[u] = quad_load<NT>(p, in.a, in.c, in.b, i0[u], nv[u]);
                    break;
                case kEltImm:
#pragma unroll
                    for (int u = 0; u < U; ++u) o[u] = f32x4{in.imm, in.imm, in.imm, in.imm};
                    break;
                case kEltStore:
                case kEltAccum:
#pragma unroll
                    for (int u = 0; u < U; ++u)
                        quad_store<NT>(p, in.a, in.c, i0[u], nv[u], y[u], in.op == kEltAccum);
                    wr = false;
                    break;
                case kEltRound: unary([&](float v) { return round_to(in.c, v); }); break;
                case kEltAdd:
#pragma unroll
                    for (int u = 0; u < U; ++u) o[u] = x[u] + y[u];
                    break;
                case kEltSub:
#pragma unroll
                    for (int u = 0; u < U; ++u) o[u] = x[u] - y[u];
                    break;
                case kEltMul:
#pragma unroll
                    for (int u = 0; u < U; ++u) o[u] = x[u] * y[u];
                    break;
                case kEltDiv:
#pragma unroll
                    for (int u = 0; u < U; ++u) o[u] = x[u] / y[u];
                    break;
                case kEltNeg:
#pragma unroll
                    for (int u = 0; u < U; ++u) o[u] = -x[u];
                    break;
                case kEltRelu: unary([](float v) { return elt_relu(v); }); break;
                case kEltGelu: unary([](float v) { return elt_gelu(v); }); break;
                case kEltElu: unary([](float v) { return elt_elu(v); }); break;
                case kEltTanh: unary([](float v) { return elt_tanh(v); }); break;
                case kEltExp: unary([](float v) { return elt_exp(v); }); break;
                case kEltLog: unary([](float v) { return elt_log(v); }); break;
                case kEltAbs: unary([](float v) { return elt_abs(v); }); break;
                case kEltReluD: unary([](float v) { return elt_relu_d(v); }); break;
                case kEltGeluD: unary([](float v) { return elt_gelu_d(v); }); break;
                case kEltEluD: unary([](float v) { return elt_elu_d(v); }); break;
                case kEltSign: unary([](float v) { return elt_sign(v); }); break;
                case kEltLabelEq:
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        f32x4 t{0.f, 0.f, 0.f, 0.f};
                        for (int e = 0; e < nv[u]; ++e) {
                            const uint64_t row = (i0[u] + e) / p.cols, col = (i0[u] + e) % p.cols;
                            t[e] = (p.labels[row] == (uint32_t)col) ? 1.0f : 0.0f;
                        }
                        o[u] = t;
                    }
                    break;
                case kEltSelect:
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const f32x4 z = get(u, in.c);
                        f32x4 t;
#pragma unroll
                        for (int e = 0; e < 4; ++e) t[e] = elt_select(x[u][e], y[u][e], z[e]);
                        o[u] = t;
                    }
                    break;
                case kEltMax:
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        f32x4 t;
#pragma unroll
                        for (int e = 0; e < 4; ++e) t[e] = elt_max(x[u][e], y[u][e]);
                        o[u] = t;
                    }
                    break;
                default: wr = false; break;
            }
            if (wr) {
#pragma unroll
                for (int u = 0; u < U; ++u) set(u, in.dst, o[u]);
            }
        }
    }
}

template <int R, int U, bool NT>
int launch_file(fg_ctx *ctx, const EltProgram &p) {
    // One pass per workgroup where the grid allows it; the launch keeps
    // gridDim.x * blockDim.x within 32 bits and the pass loop covers the
    // rest.
    uint64_t blocks = ((p.n + 3) / 4 + (uint64_t)kThreads * U - 1) / ((uint64_t)kThreads * U);
    constexpr uint64_t kMaxBlocks = (uint64_t(1) << 32) / kThreads / 2;
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    eltwise_prog_kernel<R, U, NT><<<(unsigned)blocks, kThreads, 0, ctx->stream>>>(p);
    FG_LAUNCH_CHECK("eltwise_prog_kernel");
    return FG_OK;
}

// Validates the program's indices on the host (so no kernel reads a source
// or writes a destination that was not supplied) and returns, in *live, the
// values it keeps at most at once (its registers without prefetching).
int check_program(const EltProgram &p0, int *live) {
    FG_REQUIRE(p0.n_instr >= 0 && p0.n_instr <= kEltMaxInstr, FG_ERR_INTERNAL,
               "eltwise program: %d instructions (max %d)", p0.n_instr, kEltMaxInstr);
    bool needs_cols = false;
    for (int k = 0; k < p0.n_instr; ++k) {
        const EltInstr &in = p0.ins[k];
        FG_REQUIRE(elt_reg_use(in).known, FG_ERR_INTERNAL, "eltwise program: unknown op %d", in.op);
        if (in.op == kEltLoad) {
            FG_REQUIRE(in.a < kEltMaxSrc && p0.src[in.a], FG_ERR_INTERNAL,
                       "eltwise program: load of missing source %d", in.a);
            FG_REQUIRE(in.c <= kModeScalar, FG_ERR_INTERNAL,
                       "eltwise program: bad addressing mode %d", in.c);
            FG_REQUIRE(in.b <= kBF16, FG_ERR_INTERNAL, "eltwise program: bad load type %d",
                       in.b);
            if (in.c == kModeRow) needs_cols = true;
        }
        if (in.op == kEltStore || in.op == kEltAccum) {
            FG_REQUIRE(in.a < kEltMaxDst && p0.dst[in.a], FG_ERR_INTERNAL,
                       "eltwise program: store to missing destination %d", in.a);
            FG_REQUIRE(in.c <= kBF16, FG_ERR_INTERNAL, "eltwise program: bad store type %d",
                       in.c);
        }
        if (in.op == kEltRound)
            FG_REQUIRE(in.c <= kBF16, FG_ERR_INTERNAL, "eltwise program: bad round type %d",
                       in.c);
        if (in.op == kEltLabelEq) {
            FG_REQUIRE(p0.labels, FG_ERR_INTERNAL, "eltwise program: labels missing");
            needs_cols = true;
        }
    }
    FG_REQUIRE(!needs_cols || p0.cols > 0, FG_ERR_INTERNAL, "eltwise program: cols is 0");
    EltProgram p = p0;
    char why[128] = "";
    const int regs = elt_allocate(p, false, why, sizeof why);
    FG_REQUIRE(regs >= 0, FG_ERR_INTERNAL, "eltwise program: %s", why);
    FG_REQUIRE(regs <= kEltRegs, FG_ERR_INTERNAL, "eltwise program: %d registers (max %d)",
               regs, kEltRegs);
    *live = regs;
    return FG_OK;
}

}  // namespace

// Compiles (fg_elt_jit.cpp) the kernel a launch of this program will take,
// when the mode selects one: for callers about to capture the launch.
int prepare_eltwise(fg_ctx *ctx, const EltProgram &p0) {
    if (p0.n == 0) return FG_OK;
    int live = 0;
    if (int rc = check_program(p0, &live)) return rc;
    if (!eltwise_jit_selected(p0)) return FG_OK;
    bool launched = false;
    return eltwise_jit(ctx, p0, live, true, &launched);
}

// Runs the program through its compiled kernel when the mode selects one
// (and it exists or can be built now), else through the interpreter: its
// registers allocated by liveness, on the smallest register file that holds
// them.
int launch_eltwise(fg_ctx *ctx, const EltProgram &p0) {
    if (p0.n == 0) return FG_OK;
    int live = 0;
    if (int rc = check_program(p0, &live)) return rc;
    if (eltwise_jit_selected(p0)) {
        bool launched = false;
        if (int rc = eltwise_jit(ctx, p0, live, false, &launched)) return rc;
        if (launched) return FG_OK;
    }
    eltwise_count_interpreted();
    EltProgram p = p0;
    char why[128] = "";
    int regs = elt_allocate(p, true, why, sizeof why);
    if (regs > kEltRegs) {  // prefetching raised the pressure: load in place
        p = p0;
        regs = elt_allocate(p, false, why, sizeof why);
    }
    FG_REQUIRE(regs >= 0 && regs <= kEltRegs, FG_ERR_INTERNAL, "eltwise program: %s", why);
    // Register files, from a measured sweep on tanh(a*b + c) over 8192^2
    // (3 registers): 4 registers x 3 quads 5.65 TB/s (127 VGPRs, 4 waves per
    // SIMD), 8 x 2 5.18 (125 VGPRs), 4 x 4 4.84 (163 VGPRs, 3 waves), 16 x 1
    // 4.32 (scalar-bound), 4 x 2 4.65-4.71 (an 8-entry file is indexed
    // through select chains).  Streaming accesses once each tensor is well
    // past the L2 caches (4 MiB per XCD), so small programs keep their outputs
    // cached for the next launch.
    if (p.n >= (uint64_t(1) << 22)) {
        if (regs <= 4) return launch_file<4, 3, true>(ctx, p);
        if (regs <= 8) return launch_file<8, 2, true>(ctx, p);
        return launch_file<16, 1, true>(ctx, p);
    }
    if (regs <= 4) return launch_file<4, 3, false>(ctx, p);
    if (regs <= 8) return launch_file<8, 2, false>(ctx, p);
    return launch_file<16, 1, false>(ctx, p);
}

}  // namespace fg
