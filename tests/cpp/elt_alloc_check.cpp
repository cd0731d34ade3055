// CPU check of fg::elt_allocate (ferrograd_amd/csrc/fg_eltwise.h): random
// elementwise programs are run by a scalar interpreter with the kernel's
// semantics before and after allocation, on the same data, and must give
// the same bits in every destination.  The allocated form must also use no
// register at or above the count it reports, and that count must equal the
// most values live at once when nothing is prefetched.
//
// Usage: elt_alloc_check <programs> <seed>.  Prints "OK <stats>" or the
// first failing program.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "fg_eltwise.h"

using fg::EltInstr;
using fg::EltProgram;

namespace {

constexpr uint64_t kN = 96;     // elements
constexpr uint32_t kCols = 12;  // row length

float relu(float x) { return x > 0.0f ? x : 0.0f; }

// Every op on fp32 data as the kernel computes it (the same libm calls on
// both sides of the comparison, so only register handling can differ).
float unary(int op, float x) {
    switch (op) {
        case fg::kEltNeg: return -x;
        case fg::kEltRelu: return relu(x);
        case fg::kEltGelu: return 0.5f * x * (1.0f + tanhf(0.7978846f * (x + 0.044715f * x * x * x)));
        case fg::kEltElu: return x >= 0.0f ? x : expf(x) - 1.0f;
        case fg::kEltTanh: return tanhf(x);
        case fg::kEltExp: return expf(x);
        case fg::kEltLog: return logf(x);
        case fg::kEltAbs: return fabsf(x);
        case fg::kEltReluD: return x > 0.0f ? 1.0f : 0.0f;
        case fg::kEltGeluD: return 1.0f / (1.0f + expf(-x));
        case fg::kEltEluD: return x >= 0.0f ? 1.0f : expf(x);
        case fg::kEltSign: return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
        case fg::kEltRound: return x;  // fp32 programs only
    }
    abort();
}

void run(const EltProgram &p, const uint32_t *labels) {
    for (uint64_t i = 0; i < p.n; ++i) {
        float r[fg::kEltRegs] = {};
        for (int j = 0; j < p.n_pre; ++j) r[j] = p.src[p.pre_src[j]][i];
        for (int k = 0; k < p.n_instr; ++k) {
            const EltInstr &in = p.ins[k];
            const float x = r[in.a & 15], y = r[in.b & 15];
            float o = x;
            bool wr = true;
            switch (in.op) {
                case fg::kEltLoad:
                    o = p.src[in.a][in.c == fg::kModeFull ? i
                                    : in.c == fg::kModeRow ? i % p.cols
                                                           : 0];
                    break;
                case fg::kEltImm: o = in.imm; break;
                case fg::kEltStore: p.dst[in.a][i] = y; wr = false; break;
                case fg::kEltAccum: p.dst[in.a][i] = p.dst[in.a][i] + y; wr = false; break;
                case fg::kEltAdd: o = x + y; break;
                case fg::kEltSub: o = x - y; break;
                case fg::kEltMul: o = x * y; break;
                case fg::kEltDiv: o = x / y; break;
                case fg::kEltMax: o = fmaxf(x, y); break;
                case fg::kEltLabelEq: o = labels[i / p.cols] == i % p.cols ? 1.0f : 0.0f; break;
                case fg::kEltSelect: o = x != 0.0f ? y : r[in.c & 15]; break;
                default: o = unary(in.op, x); break;
            }
            if (wr) r[in.dst] = o;
        }
    }
}

// The most values live at once: a value lives from its write to its last
// read, and an instruction's result may share a register with an operand
// that it reads last.
int max_live(const EltProgram &p) {
    std::vector<std::pair<int, int>> iv;  // [def, last read]
    std::vector<int> open(fg::kEltRegs, -1);  // index into iv of r's value
    for (int k = 0; k < p.n_instr; ++k) {
        const EltInstr &in = p.ins[k];
        const fg::EltRegUse u = fg::elt_reg_use(in);
        const int f[3] = {in.a, in.b, in.c};
        const bool use[3] = {u.a, u.b, u.c};
        for (int i = 0; i < 3; ++i)
            if (use[i]) iv[open[f[i]]].second = k;
        if (u.w) {
            iv.push_back({k, k});
            open[in.dst] = (int)iv.size() - 1;
        }
    }
    int best = 0;
    for (int k = 0; k < p.n_instr; ++k) {
        // live across the write of instruction k: defined at or before k and
        // read after k, plus the value written at k itself
        int live = 0;
        for (auto &v : iv)
            if ((v.first < k && v.second > k) || v.first == k) ++live;
        best = live > best ? live : best;
    }
    return best;
}

}  // namespace

int main(int argc, char **argv) {
    const int programs = argc > 1 ? atoi(argv[1]) : 2000;
    std::mt19937_64 rng(argc > 2 ? strtoull(argv[2], nullptr, 10) : 1);
    auto pick = [&](int n) { return (int)(rng() % (uint64_t)n); };
    const uint8_t unaries[] = {fg::kEltNeg, fg::kEltRelu, fg::kEltGelu, fg::kEltElu,
                               fg::kEltTanh, fg::kEltExp, fg::kEltAbs, fg::kEltReluD,
                               fg::kEltGeluD, fg::kEltEluD, fg::kEltSign, fg::kEltRound};
    const uint8_t binaries[] = {fg::kEltAdd, fg::kEltSub, fg::kEltMul, fg::kEltDiv, fg::kEltMax};
    // Buffers: 6 sources, 4 destinations; destination 3 is also source 5
    // (the same memory), so programs that load after storing there must not
    // have that load prefetched.  Source 4 is misaligned (never prefetched).
    constexpr int kBufFloats = kN + 8;
    std::vector<float *> mem;
    auto buf = [&]() {
        float *b = static_cast<float *>(aligned_alloc(64, kBufFloats * sizeof(float)));
        mem.push_back(b);
        return b;
    };
    uint32_t labels[kN / kCols];
    long prefetched = 0, small = 0, reduced = 0;
    for (int t = 0; t < programs; ++t) {
        float *srcb[6], *dst0[4], *dst1[4];
        for (int s = 0; s < 6; ++s) srcb[s] = buf();
        for (int d = 0; d < 4; ++d) dst0[d] = buf(), dst1[d] = buf();
        std::uniform_real_distribution<float> U(-2.0f, 2.0f);
        for (int s = 0; s < 6; ++s)
            for (int i = 0; i < kBufFloats; ++i) srcb[s][i] = U(rng);
        for (auto &l : labels) l = (uint32_t)pick(kCols);
        EltProgram p{};
        p.n = kN;
        p.cols = kCols;
        const float *src[6] = {srcb[0], srcb[1], srcb[2], srcb[3], srcb[4] + 1, srcb[5]};
        // Random straight-line program over 16 registers, every read after a
        // write of its register.
        bool written[fg::kEltRegs] = {};
        int nw = 0;
        auto any_written = [&]() {
            int r;
            do r = pick(fg::kEltRegs); while (!written[r]);
            return r;
        };
        const int len = 3 + pick(40);
        for (int k = 0; k < len; ++k) {
            EltInstr in{};
            const int kind = nw == 0 ? 0 : pick(10);
            const int dst = pick(4) == 0 && nw ? any_written() : pick(fg::kEltRegs);
            if (kind <= 2) {  // load
                in.op = fg::kEltLoad;
                in.a = (uint8_t)pick(6);
                in.b = 0;
                const int m = pick(8);
                in.c = m < 6 ? fg::kModeFull : m == 6 ? fg::kModeRow : fg::kModeScalar;
                if (in.a == 5) in.c = fg::kModeFull;  // the aliased buffer: same element only
            } else if (kind == 3) {
                in.op = pick(3) == 0 ? fg::kEltLabelEq : fg::kEltImm;
                in.imm = U(rng);
            } else if (kind <= 5) {
                in.op = pick(5) == 0 ? fg::kEltAccum : fg::kEltStore;
                in.a = (uint8_t)pick(4);
                in.b = (uint8_t)any_written();
                in.c = 0;
                p.ins[p.n_instr++] = in;
                continue;
            } else if (kind <= 7) {
                in.op = unaries[pick(sizeof unaries)];
                in.a = (uint8_t)any_written();
            } else {
                in.op = pick(6) == 0 ? fg::kEltSelect : binaries[pick(sizeof binaries)];
                in.a = (uint8_t)any_written();
                in.b = (uint8_t)any_written();
                if (in.op == fg::kEltSelect) in.c = (uint8_t)any_written();
            }
            in.dst = (uint8_t)dst;
            if (!written[dst]) written[dst] = true, ++nw;
            p.ins[p.n_instr++] = in;
        }
        // A final store of some register, so most programs write something.
        EltInstr st{};
        st.op = fg::kEltStore;
        st.a = 0;
        st.b = (uint8_t)any_written();
        p.ins[p.n_instr++] = st;

        for (int pass = 0; pass < 2; ++pass) {
            const bool pre = pass == 0;
            EltProgram a = p, b = p;
            for (int s = 0; s < 6; ++s) a.src[s] = b.src[s] = src[s];
            for (int d = 0; d < 4; ++d) a.dst[d] = dst0[d], b.dst[d] = dst1[d];
            // Destination 3 and source 5 are one buffer on each side.
            float *alias0 = buf(), *alias1 = buf();
            memcpy(alias0, srcb[5], kBufFloats * sizeof(float));
            memcpy(alias1, srcb[5], kBufFloats * sizeof(float));
            a.src[5] = alias0, a.dst[3] = alias0;
            b.src[5] = alias1, b.dst[3] = alias1;
            for (int d = 0; d < 3; ++d)
                for (int i = 0; i < kBufFloats; ++i) dst0[d][i] = dst1[d][i] = (float)(d + i);
            char why[128] = "";
            const int used = fg::elt_allocate(b, pre, why, sizeof why);
            if (used < 0) {
                printf("FAIL program %d: allocation refused: %s\n", t, why);
                return 1;
            }
            for (int k = 0; k < b.n_instr; ++k) {
                const EltInstr &in = b.ins[k];
                const fg::EltRegUse u = fg::elt_reg_use(in);
                if ((u.a && in.a >= used) || (u.b && in.b >= used) || (u.c && in.c >= used) ||
                    (u.w && in.dst >= used)) {
                    printf("FAIL program %d: register at or above the %d reported\n", t, used);
                    return 1;
                }
            }
            if (!pre && used != max_live(p)) {
                printf("FAIL program %d: %d registers for %d live values\n", t, used,
                       max_live(p));
                return 1;
            }
            run(a, labels);
            run(b, labels);
            for (int d = 0; d < 4; ++d) {
                const float *x = d == 3 ? alias0 : dst0[d], *y = d == 3 ? alias1 : dst1[d];
                if (memcmp(x, y, kBufFloats * sizeof(float)) != 0) {
                    printf("FAIL program %d (prefetch %d): destination %d differs\n", t, pre, d);
                    for (int k = 0; k < p.n_instr; ++k)
                        printf("  %2d: op %2d dst %2d a %2d b %2d c %2d\n", k, p.ins[k].op,
                               p.ins[k].dst, p.ins[k].a, p.ins[k].b, p.ins[k].c);
                    return 1;
                }
            }
            if (pre) {
                prefetched += b.n_pre > 0;
                small += used <= 4;
            } else {
                reduced += used < 16;
            }
        }
        for (float *m : mem) free(m);
        mem.clear();
    }
    printf("OK %d programs: %ld with prefetched sources, %ld in <= 4 registers, %ld below 16\n",
           programs, prefetched, small, reduced);
    return 0;
}
