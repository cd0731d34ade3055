// k_eltwise_prog.hip -- the elementwise-program kernel (see fg_eltwise.h).
// Every lane runs the same instruction stream (uniform branches), so the
// interpretation costs scalar-unit work only; the kernel stays HBM-bound
// for the short programs the planner emits.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "fg_act.h"
#include "fg_eltwise.h"
#include "fg_half.h"
#include "fg_internal.h"

namespace fg {

namespace {

constexpr int kThreads = 256;

typedef float f32x4 __attribute__((ext_vector_type(4)));

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

__device__ __forceinline__ f32x4 quad_get(const void *q, int dt, uint64_t j) {
    if (dt == kF32) return *reinterpret_cast<const f32x4 *>(static_cast<const float *>(q) + j);
    const uint2 w = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(q) + j);
    return f32x4{h16_to_f(dt, (uint16_t)(w.x & 0xffffu)), h16_to_f(dt, (uint16_t)(w.x >> 16)),
                 h16_to_f(dt, (uint16_t)(w.y & 0xffffu)), h16_to_f(dt, (uint16_t)(w.y >> 16))};
}

__device__ __forceinline__ void quad_put(void *q, int dt, uint64_t j, f32x4 v) {
    if (dt == kF32) {
        *reinterpret_cast<f32x4 *>(static_cast<float *>(q) + j) = v;
        return;
    }
    uint2 w;
    w.x = (uint32_t)f_to_h16(dt, v[0]) | ((uint32_t)f_to_h16(dt, v[1]) << 16);
    w.y = (uint32_t)f_to_h16(dt, v[2]) | ((uint32_t)f_to_h16(dt, v[3]) << 16);
    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(q) + j) = w;
}

// Source s at elements i0 .. i0+nv-1 (missing lanes of a partial quad are 0).
__device__ __forceinline__ f32x4 quad_load(const EltProgram &p, int s, int mode, int dt,
                                           uint64_t i0, int nv) {
    const void *q = p.src[s];
    if (mode == kModeScalar) {
        const float x = load_as_f(q, dt, 0);
        return f32x4{x, x, x, x};
    }
    if (mode == kModeFull) {
        if (nv == 4 && quad_aligned(q, dt)) return quad_get(q, dt, i0);
        f32x4 r{0.f, 0.f, 0.f, 0.f};
        for (int e = 0; e < nv; ++e) r[e] = load_as_f(q, dt, i0 + e);
        return r;
    }
    // Row broadcast: element i reads src[i % cols].
    const uint32_t c0 = (uint32_t)(i0 % p.cols);
    if (nv == 4 && p.cols % 4 == 0 && quad_aligned(q, dt)) return quad_get(q, dt, c0);
    f32x4 r{0.f, 0.f, 0.f, 0.f};
    for (int e = 0; e < nv; ++e) r[e] = load_as_f(q, dt, (c0 + (uint32_t)e) % p.cols);
    return r;
}

__device__ __forceinline__ void quad_store(const EltProgram &p, int d, int dt, uint64_t i0, int nv,
                                           f32x4 v, bool accum) {
    void *q = p.dst[d];
    if (nv == 4 && quad_aligned(q, dt)) {
        if (accum) v += quad_get(q, dt, i0);
        quad_put(q, dt, i0, v);
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

template <int N>
using QIdx = std::integral_constant<int, N>;
// f(QIdx<0>{}), ..., f(QIdx<Q-1>{}): per-quad code with a constant quad index.
template <int Q, class F>
__device__ __forceinline__ void for_quads(F &&f) {
    static_assert(Q == 1 || Q == 2, "one or two quads per thread");
    f(QIdx<0>{});
    if constexpr (Q > 1) f(QIdx<1>{});
}

// Q: quads per thread and pass.  Every lane runs the same instruction
// stream, so decoding an instruction, branching on its op and reading its
// pointers is scalar work done once per wave and pass; the scalar unit is
// shared by the CU's waves and is what bounds short programs (tanh(a*b + c):
// ~500 scalar instructions per wave, 60 % of the kernel's cycles).  Thread t
// of a workgroup takes quads base + q * kThreads + t (q < Q), so each load
// and store of the pass stays coalesced.  The pass loop is uniform: a lane
// past the end takes an empty quad (loads give 0, stores skip), so the
// interpreter runs outside any divergent region.
template <int Q>
__global__ __launch_bounds__(kThreads) void eltwise_prog_kernel(const EltProgram p) {
    const uint64_t nq = (p.n + 3) / 4;
    const uint64_t span = (uint64_t)kThreads * Q;
    const uint64_t stride = (uint64_t)gridDim.x * span;
    for (uint64_t base = (uint64_t)blockIdx.x * span; base < nq; base += stride) {
        uint64_t i0[Q];
        int nv[Q];  // elements of quad q (0 past the end: loads give 0, stores skip)
        // The register file: an array per element of each quad, all indexed
        // by the same uniform register number.  Every access names its array
        // at compile time (the quad through get / set, the element by name),
        // which keeps each array in VGPRs, read and written through indexed
        // moves; a float4 array, or one indexed by a run-time quad, would go
        // to scratch memory.
        float a0[kEltRegs], a1[kEltRegs], a2[kEltRegs], a3[kEltRegs];  // quad 0
        float b0[kEltRegs], b1[kEltRegs], b2[kEltRegs], b3[kEltRegs];  // quad 1 (Q = 2)
        auto get = [&](auto qc, int k) {
            k &= kEltRegs - 1;
            if constexpr (decltype(qc)::value == 0) return f32x4{a0[k], a1[k], a2[k], a3[k]};
            else return f32x4{b0[k], b1[k], b2[k], b3[k]};
        };
        auto set = [&](auto qc, int k, f32x4 v) {
            k &= kEltRegs - 1;
            if constexpr (decltype(qc)::value == 0) {
                a0[k] = v[0];
                a1[k] = v[1];
                a2[k] = v[2];
                a3[k] = v[3];
            } else {
                b0[k] = v[0];
                b1[k] = v[1];
                b2[k] = v[2];
                b3[k] = v[3];
            }
        };
        // The prefetched sources' quads, all loads issued before the program
        // runs: a load's value must be present when it is written to the
        // register file (indexed at run time), so loads issued by the
        // program itself each wait for their data in turn.
        constexpr f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 pre[Q][kEltPre];
        for_quads<Q>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            const uint64_t qi = base + (uint64_t)q * kThreads + threadIdx.x;
            i0[q] = 4 * qi;
            nv[q] = qi >= nq ? 0 : (p.n - i0[q] >= 4 ? 4 : (int)(p.n - i0[q]));
#pragma unroll
            for (int k = 0; k < kEltRegs; ++k) set(qc, k, zero);
#pragma unroll
            for (int j = 0; j < kEltPre; ++j)
                pre[q][j] = (j < p.n_pre && nv[q] == 4)
                                ? *reinterpret_cast<const f32x4 *>(p.src[p.pre_src[j]] + i0[q])
                                : zero;
        });
        for (int k = 0; k < p.n_instr; ++k) {
            const EltInstr in = p.ins[k];
            // One read site for the operands and one write site for the
            // result (each indexed access costs scalar work to set up, and
            // more sites hold more registers).
            f32x4 x[Q], y[Q], o[Q];
            for_quads<Q>([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                x[q] = get(qc, in.a);
                y[q] = get(qc, in.b);
                o[q] = x[q];
            });
            bool wr = true;  // the instruction writes register in.dst
            auto unary = [&](auto f) {
#pragma unroll
                for (int q = 0; q < Q; ++q) o[q] = quad_map(x[q], f);
            };
            switch (in.op) {
                case kEltLoad:
#pragma unroll
                    for (int q = 0; q < Q; ++q) {
                        if (in.pre && nv[q] == 4) {
                            switch (in.pre) {  // a constant index into pre[q]
                                case 1: o[q] = pre[q][0]; break;
                                case 2: o[q] = pre[q][1]; break;
                                case 3: o[q] = pre[q][2]; break;
                                default: o[q] = pre[q][3]; break;
                            }
                        } else {
                            o[q] = quad_load(p, in.a, in.c, in.b, i0[q], nv[q]);
                        }
                    }
                    break;
                case kEltImm:
#pragma unroll
                    for (int q = 0; q < Q; ++q) o[q] = f32x4{in.imm, in.imm, in.imm, in.imm};
                    break;
                case kEltStore:
                case kEltAccum:
#pragma unroll
                    for (int q = 0; q < Q; ++q)
                        quad_store(p, in.a, in.c, i0[q], nv[q], y[q], in.op == kEltAccum);
                    wr = false;
                    break;
                case kEltRound: unary([&](float v) { return round_to(in.c, v); }); break;
                case kEltAdd:
#pragma unroll
                    for (int q = 0; q < Q; ++q) o[q] = x[q] + y[q];
                    break;
                case kEltSub:
#pragma unroll
                    for (int q = 0; q < Q; ++q) o[q] = x[q] - y[q];
                    break;
                case kEltMul:
#pragma unroll
                    for (int q = 0; q < Q; ++q) o[q] = x[q] * y[q];
                    break;
                case kEltDiv:
#pragma unroll
                    for (int q = 0; q < Q; ++q) o[q] = x[q] / y[q];
                    break;
                case kEltNeg:
#pragma unroll
                    for (int q = 0; q < Q; ++q) o[q] = -x[q];
                    break;
                case kEltRelu: unary([](float v) { return act_fwd(kActRelu, v); }); break;
                case kEltGelu: unary([](float v) { return act_fwd(kActGelu, v); }); break;
                case kEltElu: unary([](float v) { return v >= 0.0f ? v : expf(v) - 1.0f; }); break;
                case kEltTanh: unary([](float v) { return tanhf(v); }); break;
                case kEltExp: unary([](float v) { return expf(v); }); break;
                case kEltLog: unary([](float v) { return logf(v); }); break;
                case kEltAbs: unary([](float v) { return fabsf(v); }); break;
                case kEltReluD: unary([](float v) { return act_grad(kActRelu, v); }); break;
                case kEltGeluD: unary([](float v) { return act_grad(kActGelu, v); }); break;
                case kEltEluD: unary([](float v) { return v >= 0.0f ? 1.0f : expf(v); }); break;
                case kEltSign:
                    unary([](float v) { return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f); });
                    break;
                case kEltLabelEq:
#pragma unroll
                    for (int q = 0; q < Q; ++q) {
                        f32x4 t{0.f, 0.f, 0.f, 0.f};
                        for (int e = 0; e < nv[q]; ++e) {
                            const uint64_t row = (i0[q] + e) / p.cols, col = (i0[q] + e) % p.cols;
                            t[e] = (p.labels[row] == (uint32_t)col) ? 1.0f : 0.0f;
                        }
                        o[q] = t;
                    }
                    break;
                case kEltSelect:
                    for_quads<Q>([&](auto qc) {
                        constexpr int q = decltype(qc)::value;
                        const f32x4 z = get(qc, in.c);
                        f32x4 t;
#pragma unroll
                        for (int e = 0; e < 4; ++e) t[e] = x[q][e] != 0.0f ? y[q][e] : z[e];
                        o[q] = t;
                    });
                    break;
                case kEltMax:
#pragma unroll
                    for (int q = 0; q < Q; ++q) {
                        f32x4 t;
#pragma unroll
                        for (int e = 0; e < 4; ++e) t[e] = fmaxf(x[q][e], y[q][e]);
                        o[q] = t;
                    }
                    break;
                default: wr = false; break;
            }
            if (wr) for_quads<Q>([&](auto qc) { set(qc, in.dst, o[decltype(qc)::value]); });
        }
    }
}

}  // namespace

// Validates the program's indices on the host (so the kernel never reads a
// source or writes a destination that was not supplied) and launches it.
int launch_eltwise(fg_ctx *ctx, const EltProgram &p0) {
    if (p0.n == 0) return FG_OK;
    // Prefetch slots for up to kEltPre sources read whole as fp32 from
    // 16-byte aligned memory (a source read by several loads takes one).
    EltProgram p = p0;
    p.n_pre = 0;
    for (int k = 0; k < p.n_instr && k < kEltMaxInstr; ++k) {
        EltInstr &in = p.ins[k];
        in.pre = 0;
        if (in.op != kEltLoad || in.c != kModeFull || in.b != kF32 || in.a >= kEltMaxSrc ||
            !p.src[in.a] || (((uintptr_t)p.src[in.a]) & 15u) != 0)
            continue;
        int slot = -1;
        for (int j = 0; j < p.n_pre; ++j)
            if (p.pre_src[j] == in.a) slot = j;
        if (slot < 0 && p.n_pre < kEltPre) {
            slot = p.n_pre++;
            p.pre_src[slot] = in.a;
        }
        if (slot >= 0) in.pre = (uint8_t)(slot + 1);
    }
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
    // One quad per thread and as many workgroups as that takes, up to the
    // grid limit (a capped grid looping over the tensor streamed at a
    // fraction of the rate); the kernel's loop covers anything beyond.
    uint64_t blocks = ((p.n + 3) / 4 + kThreads - 1) / kThreads;
    if (blocks > (1u << 30)) blocks = 1u << 30;
#ifndef FG_ELT_QUADS  // quads per thread and pass (a knob for measurement builds)
#define FG_ELT_QUADS 1
#endif
    constexpr int kQ = FG_ELT_QUADS;
    blocks = (blocks + kQ - 1) / kQ;
    eltwise_prog_kernel<kQ><<<(unsigned)blocks, kThreads, 0, ctx->stream>>>(p);
    FG_LAUNCH_CHECK("eltwise_prog_kernel");
    return FG_OK;
}

}  // namespace fg
