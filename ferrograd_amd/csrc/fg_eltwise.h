// fg_eltwise.h -- elementwise program: a tiny register machine evaluated per
// element by one kernel launch.  The planner compiles fused chains of
// ferrograd-nn elementwise ops (forward and backward) and the MSE / BCE /
// CE-on-probabilities losses into these programs, so arbitrary chains run
// as single launches from ahead-of-time code (the reference instead emits a
// new HIP source per fused kernel and compiles it with hipRTC,
// rocm/generate.rs:17-70).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>

namespace fg {

enum EltOp : uint8_t {
    kEltLoad = 0,   // r[dst] = src[a] at the element, addressing mode c, element type b
    kEltImm,        // r[dst] = imm
    kEltStore,      // dsts[a][i] = r[b]              (element type c, rounded to it)
    kEltAccum,      // dsts[a][i] = dsts[a][i] + r[b]  (element type c, rounded to it)
    kEltAdd,        // r[dst] = r[a] + r[b]
    kEltSub,
    kEltMul,
    kEltDiv,
    kEltNeg,        // r[dst] = -r[a]
    kEltRelu,
    kEltGelu,
    kEltElu,        // x >= 0 ? x : exp(x) - 1   (unary.rs:329-434)
    kEltTanh,
    kEltExp,
    kEltLog,
    kEltAbs,
    kEltReluD,      // [x > 0]
    kEltGeluD,      // d gelu / dx
    kEltEluD,       // x >= 0 ? 1 : exp(x)
    kEltSign,       // x > 0 ? 1 : (x < 0 ? -1 : 0)
    kEltLabelEq,    // r[dst] = (col == labels[row]) ? 1 : 0
    kEltSelect,     // r[dst] = r[a] != 0 ? r[b] : r[c]
    kEltMax,        // r[dst] = max(r[a], r[b])
    kEltRound,      // r[dst] = r[a] rounded to element type c (a 16-bit node value)
};

// Source addressing modes.
enum EltMode : uint8_t {
    kModeFull = 0,  // src[i]
    kModeRow = 1,   // src[i % cols]   (row-broadcast bias vector)
    kModeScalar = 2 // src[0]
};

constexpr int kEltMaxInstr = 64;
constexpr int kEltMaxSrc = 12;
constexpr int kEltMaxDst = 8;
constexpr int kEltRegs = 16;
constexpr int kEltPre = 4;  // sources prefetched per quad (launch_eltwise)

// Register operands by op: a and b of binary ops and kEltMax, a of unary ops
// and kEltRound, b of a store / accumulate, a, b and c of kEltSelect; dst of
// every op but a store / accumulate.  Other fields are not registers.
struct EltInstr {
    uint8_t op, dst, a, b, c, pad[3];
    float imm;
};

// Element types (b of a load, c of a store / accumulate / round) are the
// fg_half.h codes: 0 fp32, 1 fp16, 2 bf16.  16-bit sources and destinations
// are addressed as 16-bit words through the same pointer arrays.

// Passed by value as the kernel argument.  Every field the kernel indexes
// with a run-time value (src, dst, ins) has elements of at least 4 bytes:
// the compiler may reuse a computed element address as the base of a scalar
// (SMEM) load, and SMEM ignores the low two address bits, so an array of
// bytes indexed next to the pointer array once produced misaligned pointer
// reads.  The addressing mode of a load therefore travels in the
// instruction (field c), not in a byte array.
struct EltProgram {
    const float *src[kEltMaxSrc];
    float *dst[kEltMaxDst];
    const uint32_t *labels;
    uint64_t n;     // elements
    uint32_t cols;  // row length (for row-broadcast and labels)
    int32_t n_instr;
    EltInstr ins[kEltMaxInstr];
    // Filled by launch_eltwise: the sources whose quads every thread loads
    // into registers 0 .. n_pre-1 before running the program (whole-tensor
    // sources of element type pre_dt[j], aligned for quad loads, disjoint
    // from every destination), their loads taken out of the program.
    int32_t n_pre;
    int32_t pre_src[kEltPre];
    int32_t pre_dt[kEltPre];
};

// The rule above, checked: every array the kernel indexes with a run-time
// value has elements of a whole number of 4-byte words, at a 4-byte aligned
// offset, so no scalar load of one can start at a byte address.
static_assert(sizeof(EltProgram::src[0]) % 4 == 0 && offsetof(EltProgram, src) % 4 == 0,
              "src[] elements must be whole 4-byte words");
static_assert(sizeof(EltProgram::dst[0]) % 4 == 0 && offsetof(EltProgram, dst) % 4 == 0,
              "dst[] elements must be whole 4-byte words");
static_assert(sizeof(EltInstr) % 4 == 0 && alignof(EltInstr) >= 4 &&
                  offsetof(EltProgram, ins) % 4 == 0,
              "ins[] elements must be whole 4-byte words");

// ---------------------------------------------------------------- host side
// (plain C++: the launch code and the CPU tests of the allocation use it)

// Which fields of an instruction are registers.
struct EltRegUse {
    bool a, b, c, w;
    bool known;  // a valid op
};

inline EltRegUse elt_reg_use(const EltInstr &in) {
    switch (in.op) {
        case kEltLoad: case kEltImm: case kEltLabelEq: return {false, false, false, true, true};
        case kEltStore: case kEltAccum: return {false, true, false, false, true};
        case kEltRound: case kEltNeg: case kEltRelu: case kEltGelu: case kEltElu: case kEltTanh:
        case kEltExp: case kEltLog: case kEltAbs: case kEltReluD: case kEltGeluD: case kEltEluD:
        case kEltSign:
            return {true, false, false, true, true};
        case kEltAdd: case kEltSub: case kEltMul: case kEltDiv: case kEltMax:
            return {true, true, false, true, true};
        case kEltSelect: return {true, true, true, true, true};
        default: return {false, false, false, false, false};
    }
}

// Element size of a storage type code (0 fp32, 1 fp16, 2 bf16).
inline uint64_t elt_esize(int dt) { return dt == 0 ? 4 : 2; }

// Rewrites a validated program into the form the kernel runs:
//  * prefetch (when `prefetch`): up to kEltPre sources loaded whole (mode
//    kModeFull) from memory aligned for quad loads (16 bytes fp32, 8 bytes
//    16-bit) and disjoint from every destination's bytes (so no store of the
//    program can precede a load of the same memory) are bound to registers
//    0 .. n_pre-1 (n_pre, pre_src, pre_dt) and their loads removed;
//  * registers by liveness: each write starts a new value, and a register
//    is free again once its value's last reader has run.  An instruction
//    reads its operands before it writes, so its result may take the
//    register of an operand it reads last.  For straight-line code this
//    linear scan uses exactly as many registers as values live at once.
// Returns the registers used (possibly above kEltRegs when prefetching
// raised the pressure; the caller then allocates again without it), or -1
// with `why` set when an instruction reads a register never written.
inline int elt_allocate(EltProgram &p, bool prefetch, char *why, size_t why_len) {
    const int n = p.n_instr;
    int pre_of_src[kEltMaxSrc];
    for (int s = 0; s < kEltMaxSrc; ++s) pre_of_src[s] = -1;
    p.n_pre = 0;
    if (prefetch) {
        for (int k = 0; k < n; ++k) {
            const EltInstr &in = p.ins[k];
            if (in.op != kEltLoad || in.c != kModeFull || in.a >= kEltMaxSrc ||
                pre_of_src[in.a] >= 0 || p.n_pre == kEltPre)
                continue;
            const uintptr_t lo = (uintptr_t)p.src[in.a];
            if ((lo & (in.b == 0 ? 15u : 7u)) != 0) continue;
            const uintptr_t hi = lo + p.n * elt_esize(in.b);
            bool clash = false;
            for (int j = 0; j < n && !clash; ++j) {
                const EltInstr &st = p.ins[j];
                if (st.op != kEltStore && st.op != kEltAccum) continue;
                const uintptr_t dlo = (uintptr_t)p.dst[st.a];
                const uintptr_t dhi = dlo + p.n * elt_esize(st.c);
                clash = dlo < hi && lo < dhi;
            }
            if (clash) continue;
            pre_of_src[in.a] = p.n_pre;
            p.pre_src[p.n_pre] = in.a;
            p.pre_dt[p.n_pre] = in.b;
            ++p.n_pre;
        }
    }
    // Values 0 .. n_pre-1 are the prefetched sources, then one per write;
    // cur[r] = the value register r holds (-1: never written).
    constexpr int kMaxVals = kEltPre + kEltMaxInstr;
    int cur[kEltRegs];
    for (int r = 0; r < kEltRegs; ++r) cur[r] = -1;
    int nvals = p.n_pre;
    int last_use[kMaxVals];
    for (int v = 0; v < kMaxVals; ++v) last_use[v] = -1;
    int rd[kEltMaxInstr][3], wv[kEltMaxInstr];
    bool keep[kEltMaxInstr];
    for (int k = 0; k < n; ++k) {
        const EltInstr &in = p.ins[k];
        const EltRegUse u = elt_reg_use(in);
        const uint8_t f[3] = {in.a, in.b, in.c};
        const bool use[3] = {u.a, u.b, u.c};
        for (int i = 0; i < 3; ++i) {
            rd[k][i] = -1;
            if (!use[i]) continue;
            const int v = f[i] < kEltRegs ? cur[f[i]] : -1;
            if (v < 0) {
                snprintf(why, why_len, "instruction %d reads register %d before any write", k,
                         f[i]);
                return -1;
            }
            rd[k][i] = v;
            last_use[v] = k;
        }
        keep[k] = !(in.op == kEltLoad && in.c == kModeFull && in.a < kEltMaxSrc &&
                    pre_of_src[in.a] >= 0 && p.pre_dt[pre_of_src[in.a]] == in.b);
        wv[k] = -1;
        if (u.w) {
            if (in.dst >= kEltRegs) {
                snprintf(why, why_len, "instruction %d writes register %d", k, in.dst);
                return -1;
            }
            wv[k] = keep[k] ? nvals++ : pre_of_src[in.a];
            cur[in.dst] = wv[k];
        }
    }
    int phys[kMaxVals];
    bool busy[kMaxVals] = {};  // at most kMaxVals values, so registers < kMaxVals
    int used = p.n_pre;
    for (int v = 0; v < p.n_pre; ++v) {
        phys[v] = v;
        busy[v] = last_use[v] >= 0;
    }
    int out = 0;
    for (int k = 0; k < n; ++k) {
        for (int i = 0; i < 3; ++i)  // operands whose last reader this is
            if (rd[k][i] >= 0 && last_use[rd[k][i]] == k) busy[phys[rd[k][i]]] = false;
        if (!keep[k]) continue;
        EltInstr in = p.ins[k];
        if (rd[k][0] >= 0) in.a = (uint8_t)phys[rd[k][0]];
        if (rd[k][1] >= 0) in.b = (uint8_t)phys[rd[k][1]];
        if (rd[k][2] >= 0) in.c = (uint8_t)phys[rd[k][2]];
        if (wv[k] >= 0) {
            int r = 0;
            while (busy[r]) ++r;
            phys[wv[k]] = r;
            busy[r] = last_use[wv[k]] > k;  // a value nobody reads frees at once
            if (r + 1 > used) used = r + 1;
            in.dst = (uint8_t)r;
        }
        p.ins[out++] = in;
    }
    p.n_instr = out;
    return used;
}

}  // namespace fg
