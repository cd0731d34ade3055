// fg_elt_jit.h -- the HIP source of a compiled elementwise kernel: one
// elementwise program (fg_eltwise.h) written out as straight-line code and
// compiled at run time with hipRTC (fg_elt_jit.cpp), as the reference
// compiles each fused kernel it generates (rocm/generate.rs:17-70,
// rocm/mod.rs:140-170).  Host-only, plain C++: the library and the CPU test
// that compiles generated programs (tests/cpp/elt_jit_check.cpp) use it.
//
// The kernel evaluates what the interpreter (k_eltwise_prog.hip) evaluates,
// bit for bit: the same thread -> quad mapping and memory accesses, each op
// through the shared definition of fg_elt_ops.h, and every op's result
// passed through an empty inline-assembly barrier.  The barrier keeps each
// op a separate rounding point as in the interpreter, whose values pass
// through its register file: without it the compiler could contract a
// multiply ending one op with an add starting the next into one fma, or
// fold a constant through a transcendental at compile time.
//
// Differences from the interpreter are all in what the compiler is told:
// the values live in registers named at compile time (no register file to
// index, no instruction decoding), loads of memory that no store of the
// program touches (checked on the host, as for the interpreter's prefetch)
// are issued before the program, scalar sources and immediates are read
// once per thread, and pointer alignment is part of the generated code.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "fg_eltwise.h"

namespace fg {

// The kernel's argument, by value (the generated source declares the same
// layout: pointers, then n, then cols).
struct EltJitArgs {
    const void *src[kEltMaxSrc];
    void *dst[kEltMaxDst];
    const uint32_t *labels;
    uint64_t n;
    uint32_t cols;
};

static_assert(sizeof(EltJitArgs) == 184 && offsetof(EltJitArgs, labels) == 160 &&
                  offsetof(EltJitArgs, n) == 168 && offsetof(EltJitArgs, cols) == 176,
              "the generated kernels' Args layout");

// What a generated kernel is specialised on besides its instructions.
struct EltJitShape {
    int quads = 1;          // quads per thread and pass (1, 2 or 4)
    bool nt = false;        // non-temporal loads and stores (large tensors)
    uint32_t src_al = 0;    // bit k: src[k] aligned for quad access
    uint32_t dst_al = 0;    // bit k: dst[k] aligned for quad access
    bool cols4 = false;     // cols % 4 == 0 (row-broadcast quads)
};

constexpr const char *kEltJitKernel = "fg_elt_kernel";

// Device helpers of every generated kernel, after the shared headers.
inline const char *elt_jit_prelude() {
    return R"FGJIT(
typedef __hip_internal::uint16_t uint16_t;
typedef __hip_internal::uint32_t uint32_t;
typedef __hip_internal::uint64_t uint64_t;
#include "fg_elt_ops.h"
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
namespace fgj {
using namespace fg;
// An op's result, opaque to the optimiser (no contraction or folding across it).
__device__ __forceinline__ f32x4 bar(f32x4 v) { asm("" : "+v"(v)); return v; }
template <int DT, bool NT>
__device__ __forceinline__ f32x4 get4(const void *q, uint64_t j) {
    if (DT == kF32) {
        const f32x4 *a = reinterpret_cast<const f32x4 *>(static_cast<const float *>(q) + j);
        return NT ? __builtin_nontemporal_load(a) : *a;
    }
    const u32x2 *a = reinterpret_cast<const u32x2 *>(static_cast<const uint16_t *>(q) + j);
    const u32x2 w = NT ? __builtin_nontemporal_load(a) : *a;
    return f32x4{h16_to_f(DT, (uint16_t)(w.x & 0xffffu)), h16_to_f(DT, (uint16_t)(w.x >> 16)),
                 h16_to_f(DT, (uint16_t)(w.y & 0xffffu)), h16_to_f(DT, (uint16_t)(w.y >> 16))};
}
template <int DT, bool NT>
__device__ __forceinline__ void put4(void *q, uint64_t j, f32x4 v) {
    if (DT == kF32) {
        f32x4 *a = reinterpret_cast<f32x4 *>(static_cast<float *>(q) + j);
        if (NT) __builtin_nontemporal_store(v, a); else *a = v;
        return;
    }
    u32x2 w;
    w.x = (uint32_t)f_to_h16(DT, v[0]) | ((uint32_t)f_to_h16(DT, v[1]) << 16);
    w.y = (uint32_t)f_to_h16(DT, v[2]) | ((uint32_t)f_to_h16(DT, v[3]) << 16);
    u32x2 *a = reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(q) + j);
    if (NT) __builtin_nontemporal_store(w, a); else *a = w;
}
template <int DT, bool NT, bool AL>
__device__ __forceinline__ f32x4 ld_full(const void *q, uint64_t i0, int nv) {
    if (AL && nv == 4) return get4<DT, NT>(q, i0);
    f32x4 r{0.f, 0.f, 0.f, 0.f};
    for (int e = 0; e < nv; ++e) r[e] = load_as_f(q, DT, i0 + e);
    return r;
}
template <int DT, bool AL>
__device__ __forceinline__ f32x4 ld_row(const void *q, uint64_t i0, int nv, uint32_t cols) {
    const uint32_t c0 = (uint32_t)(i0 % cols);
    if (AL && nv == 4) return get4<DT, false>(q, c0);
    f32x4 r{0.f, 0.f, 0.f, 0.f};
    for (int e = 0; e < nv; ++e) r[e] = load_as_f(q, DT, (c0 + (uint32_t)e) % cols);
    return r;
}
template <int DT>
__device__ __forceinline__ f32x4 ld_scalar(const void *q) {
    const float x = load_as_f(q, DT, 0);
    return f32x4{x, x, x, x};
}
template <int DT, bool NT, bool AL, bool ACC>
__device__ __forceinline__ void st(void *q, uint64_t i0, int nv, f32x4 v) {
    if (AL && nv == 4) {
        if (ACC) v += get4<DT, NT>(q, i0);
        put4<DT, NT>(q, i0, v);
        return;
    }
    for (int e = 0; e < nv; ++e)
        store_from_f(q, DT, i0 + e, ACC ? load_as_f(q, DT, i0 + e) + v[e] : v[e]);
}
__device__ __forceinline__ f32x4 label_eq(const uint32_t *labels, uint64_t i0, int nv,
                                          uint32_t cols) {
    f32x4 t{0.f, 0.f, 0.f, 0.f};
    for (int e = 0; e < nv; ++e) {
        const uint64_t row = (i0 + e) / cols, col = (i0 + e) % cols;
        t[e] = (labels[row] == (uint32_t)col) ? 1.0f : 0.0f;
    }
    return t;
}
template <class F>
__device__ __forceinline__ f32x4 map(f32x4 x, F f) {
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = f(x[e]);
    return r;
}
template <int DT>
__device__ __forceinline__ f32x4 round4(f32x4 x) {
    return map(x, [](float v) { return round_to(DT, v); });
}
__device__ __forceinline__ f32x4 sel4(f32x4 c, f32x4 t, f32x4 f) {
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = elt_select(c[e], t[e], f[e]);
    return r;
}
__device__ __forceinline__ f32x4 max4(f32x4 a, f32x4 b) {
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = elt_max(a[e], b[e]);
    return r;
}
struct Args {
    const void *src[12];
    void *dst[8];
    const uint32_t *labels;
    uint64_t n;
    uint32_t cols;
};
static_assert(sizeof(Args) == 184 && __builtin_offsetof(Args, labels) == 160 &&
                  __builtin_offsetof(Args, n) == 168 && __builtin_offsetof(Args, cols) == 176,
              "the host's EltJitArgs layout");
}  // namespace fgj
)FGJIT";
}

// The shared-header function of a unary op ("" if op is not unary).
inline const char *elt_jit_unary_fn(int op) {
    switch (op) {
        case kEltRelu: return "fg::elt_relu";
        case kEltGelu: return "fg::elt_gelu";
        case kEltElu: return "fg::elt_elu";
        case kEltTanh: return "fg::elt_tanh";
        case kEltExp: return "fg::elt_exp";
        case kEltLog: return "fg::elt_log";
        case kEltAbs: return "fg::elt_abs";
        case kEltReluD: return "fg::elt_relu_d";
        case kEltGeluD: return "fg::elt_gelu_d";
        case kEltEluD: return "fg::elt_elu_d";
        case kEltSign: return "fg::elt_sign";
        default: return "";
    }
}

// Quads per thread and pass for a program that keeps `live` values (its
// register count after allocation): every value of every quad stays in
// registers, so the quads multiply the registers a thread holds, and fewer
// registers let more waves keep loads in flight.  Measured (HIP events, one
// process): tanh(a*b + c) over 8192^2 (3 values) 0.266 / 0.258 / 0.258 ms
// with 4 / 2 / 1 quads (interpreter 0.289); the seven-input expression
// ((a*b + c*d)(e - f)) / (g*g + 1) over 4096 x 8192, forward 0.389 / 0.382 /
// 0.389 ms (interpreter 0.429), its backward's programs 0.742 / 0.726 /
// 0.715 ms (interpreter 0.808).
inline int elt_jit_quads(int live) { return live <= 4 ? 2 : 1; }

// The kernel source of a validated program (launch_eltwise's checks: known
// ops, sources, destinations and element types present, registers written
// before they are read).  Returns "" with `why` set on a program it cannot
// express.
inline std::string elt_jit_source(const EltProgram &p, const EltJitShape &s, char *why,
                                  size_t why_len) {
    static_assert(kEltMaxSrc == 12 && kEltMaxDst == 8, "the generated Args layout");
    const int n = p.n_instr;
    // Memory a store or accumulate of the program writes: loads of other
    // memory may go ahead of the program.
    auto writes = [&](uintptr_t lo, uintptr_t hi) {
        for (int j = 0; j < n; ++j) {
            const EltInstr &st = p.ins[j];
            if (st.op != kEltStore && st.op != kEltAccum) continue;
            const uintptr_t dlo = (uintptr_t)p.dst[st.a];
            const uintptr_t dhi = dlo + p.n * elt_esize(st.c);
            if (dlo < hi && lo < dhi) return true;
        }
        return false;
    };
    auto extent = [&](const EltInstr &in) {  // bytes a load reads
        const uint64_t count = in.c == kModeFull ? p.n : in.c == kModeRow ? p.cols : 1;
        return count * elt_esize(in.b);
    };
    auto flt = [](float f) {  // the exact bits of an fp32 constant
        uint32_t u;
        memcpy(&u, &f, 4);
        char b[40];
        snprintf(b, sizeof b, "__uint_as_float(0x%08xu)", u);
        return std::string(b);
    };
    const std::string U = std::to_string(s.quads);
    const char *NT = s.nt ? "true" : "false";
    std::string outer, pass, body;  // before the pass loop, hoisted loads, the program
    int cur[kEltRegs];
    for (int r = 0; r < kEltRegs; ++r) cur[r] = -1;
    int nvals = 0;
    auto val = [&](int reg, int k) -> std::string {
        if (reg >= kEltRegs || cur[reg] < 0) {
            snprintf(why, why_len, "instruction %d reads register %d before any write", k, reg);
            return "";
        }
        return "v" + std::to_string(cur[reg]);
    };
    auto each = [&](std::string &dst, const std::string &stmt) {
        dst += "#pragma unroll\n    for (int u = 0; u < " + U + "; ++u) " + stmt + "\n    ";
    };
    for (int k = 0; k < n; ++k) {
        const EltInstr &in = p.ins[k];
        const EltRegUse use = elt_reg_use(in);
        if (!use.known) {
            snprintf(why, why_len, "instruction %d: unknown op %d", k, in.op);
            return "";
        }
        std::string a, b, c;
        if (use.a && (a = val(in.a, k)).empty()) return "";
        if (use.b && (b = val(in.b, k)).empty()) return "";
        if (use.c && (c = val(in.c, k)).empty()) return "";
        if (in.op == kEltStore || in.op == kEltAccum) {
            const bool al = (s.dst_al >> in.a) & 1u;
            each(body, "fgj::st<" + std::to_string(in.c) + ", " + NT + ", " +
                           (al ? "true" : "false") + ", " +
                           (in.op == kEltAccum ? "true" : "false") + ">(a.dst[" +
                           std::to_string(in.a) + "], i0[u], nv[u], " + b + "[u]);");
            continue;
        }
        if (in.dst >= kEltRegs) {
            snprintf(why, why_len, "instruction %d writes register %d", k, in.dst);
            return "";
        }
        const std::string v = "v" + std::to_string(nvals);
        if (in.op == kEltImm) {
            outer += "const f32x4 " + v + "_1 = fgj::bar(f32x4{" + flt(in.imm) + ", " +
                     flt(in.imm) + ", " + flt(in.imm) + ", " + flt(in.imm) + "});\n    ";
            outer += "f32x4 " + v + "[" + U + "];\n    ";
            each(outer, v + "[u] = " + v + "_1;");
        } else if (in.op == kEltLoad) {
            const std::string dt = std::to_string(in.b), src = "a.src[" + std::to_string(in.a) + "]";
            const bool al = (s.src_al >> in.a) & 1u;
            const uintptr_t lo = (uintptr_t)p.src[in.a];
            const bool early = !writes(lo, lo + extent(in));
            if (in.c == kModeScalar) {
                std::string &to = early ? outer : body;
                to += "f32x4 " + v + "[" + U + "];\n    ";
                each(to, v + "[u] = fgj::ld_scalar<" + dt + ">(" + src + ");");
            } else {
                std::string &to = early ? pass : body;
                to += "f32x4 " + v + "[" + U + "];\n    ";
                if (in.c == kModeFull)
                    each(to, v + "[u] = fgj::ld_full<" + dt + ", " + NT + ", " +
                                 (al ? "true" : "false") + ">(" + src + ", i0[u], nv[u]);");
                else
                    each(to, v + "[u] = fgj::ld_row<" + dt + ", " +
                                 (al && s.cols4 ? "true" : "false") + ">(" + src +
                                 ", i0[u], nv[u], a.cols);");
            }
        } else {
            std::string e;
            switch (in.op) {
                case kEltAdd: e = a + "[u] + " + b + "[u]"; break;
                case kEltSub: e = a + "[u] - " + b + "[u]"; break;
                case kEltMul: e = a + "[u] * " + b + "[u]"; break;
                case kEltDiv: e = a + "[u] / " + b + "[u]"; break;
                case kEltNeg: e = "-" + a + "[u]"; break;
                case kEltRound: e = "fgj::round4<" + std::to_string(in.c) + ">(" + a + "[u])"; break;
                case kEltLabelEq: e = "fgj::label_eq(a.labels, i0[u], nv[u], a.cols)"; break;
                case kEltSelect: e = "fgj::sel4(" + a + "[u], " + b + "[u], " + c + "[u])"; break;
                case kEltMax: e = "fgj::max4(" + a + "[u], " + b + "[u])"; break;
                default:
                    e = std::string("fgj::map(") + a + "[u], [](float t) { return " +
                        elt_jit_unary_fn(in.op) + "(t); })";
                    break;
            }
            body += "f32x4 " + v + "[" + U + "];\n    ";
            each(body, v + "[u] = fgj::bar(" + e + ");");
        }
        cur[in.dst] = nvals++;
    }
    std::string src = "#include \"fg_elt_jit_prelude.h\"\n";
    src += "extern \"C\" __global__ __launch_bounds__(256) void " + std::string(kEltJitKernel) +
           "(const fgj::Args a) {\n";
    src += "    const uint64_t nq = (a.n + 3) / 4;\n";
    src += "    const uint64_t span = 256ull * " + U + ", stride = (uint64_t)gridDim.x * span;\n";
    src += "    " + outer + "\n";
    src += "    for (uint64_t base = (uint64_t)blockIdx.x * span; base < nq; base += stride) {\n";
    src += "    uint64_t i0[" + U + "];\n    int nv[" + U + "];\n";
    src += "#pragma unroll\n    for (int u = 0; u < " + U + "; ++u) {\n";
    src += "        const uint64_t qi = base + (uint64_t)u * 256 + threadIdx.x;\n";
    src += "        i0[u] = 4 * qi;\n";
    src += "        nv[u] = qi >= nq ? 0 : (a.n - i0[u] >= 4 ? 4 : (int)(a.n - i0[u]));\n";
    src += "    }\n    " + pass + "\n    " + body + "\n    }\n}\n";
    return src;
}

}  // namespace fg
