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

// pre: set by launch_eltwise on a load it prefetches, slot + 1 (0: none).
struct EltInstr {
    uint8_t op, dst, a, b, c, pre, pad[2];
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
    // before running the program (fp32, whole tensor, 16-byte aligned).
    int32_t n_pre;
    int32_t pre_src[kEltPre];
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

}  // namespace fg
