// CPU check of the compiled elementwise kernels' source (fg::elt_jit_source,
// ferrograd_amd/csrc/fg_elt_jit.h): hipRTC compiles it for gfx950 here, no
// GPU needed.
//
// Usage: elt_jit_check <csrc dir> <out dir> <programs> <seed>
// Writes <out>/fma_bar.co and <out>/fma_nobar.co (the program a*b + c as
// generated, and with its op barriers removed) and <out>/k<i>.co for random
// programs over every op, element type, addressing mode and alignment, and
// prints "OK <programs>" or the first failure with the compiler's log.
// Usage: elt_jit_check ops <csrc dir> <out dir>
// Writes <out>/op_<name>.co: the kernel o[i] = fg::elt_<name>(a[i]) of each
// unary op, to compare with the same kernel built by hipcc.
#include <hip/hiprtc.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <random>
#include <sstream>
#include <string>
#include <vector>

#include "fg_elt_jit.h"

using fg::EltInstr;
using fg::EltProgram;

namespace {

std::string slurp(const std::string &path) {
    std::ifstream f(path);
    std::stringstream s;
    s << f.rdbuf();
    return s.str();
}

// Compiles `src` as fg_elt_jit.cpp does; false with the log on failure.
bool compile(const std::string &csrc, const std::string &src, const std::string &out) {
    static std::vector<std::string> texts;
    static std::vector<const char *> names;
    if (texts.empty()) {
        for (const char *h : {"fg_half.h", "fg_act.h", "fg_elt_ops.h"}) {
            texts.push_back(slurp(csrc + "/" + h));
            names.push_back(h);
        }
        texts.push_back(fg::elt_jit_prelude());
        names.push_back("fg_elt_jit_prelude.h");
    }
    std::vector<const char *> tp;
    for (auto &t : texts) tp.push_back(t.c_str());
    hiprtcProgram prog = nullptr;
    if (hiprtcCreateProgram(&prog, src.c_str(), "k.hip", (int)names.size(), tp.data(),
                            names.data()) != HIPRTC_SUCCESS)
        return false;
    const char *opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                          "-target-feature", "-Xclang", "-packed-fp32-ops"};
    const hiprtcResult r = hiprtcCompileProgram(prog, 7, opts);
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n + 1, '\0');
        hiprtcGetProgramLog(prog, &log[0]);
        printf("FAIL compile:\n%s\n--- source ---\n%s\n", log.c_str(), src.c_str());
        return false;
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    std::vector<char> code(n);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    std::ofstream(out, std::ios::binary).write(code.data(), (std::streamsize)n);
    return true;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc == 4 && std::string(argv[1]) == "ops") {
        for (const char *op : {"relu", "gelu", "elu", "tanh", "exp", "log", "abs", "relu_d",
                               "gelu_d", "elu_d", "sign"}) {
            const std::string src =
                std::string("typedef __hip_internal::uint16_t uint16_t;\n"
                            "typedef __hip_internal::uint32_t uint32_t;\n"
                            "typedef __hip_internal::uint64_t uint64_t;\n"
                            "#include \"fg_elt_ops.h\"\n"
                            "extern \"C\" __global__ void k(const float *a, float *o) "
                            "{ o[threadIdx.x] = fg::elt_") +
                op + "(a[threadIdx.x]); }\n";
            if (!compile(argv[2], src, std::string(argv[3]) + "/op_" + op + ".co")) return 1;
        }
        printf("OK ops\n");
        return 0;
    }
    if (argc < 5) return 2;
    const std::string csrc = argv[1], out = argv[2];
    const int programs = atoi(argv[3]);
    std::mt19937_64 rng(strtoull(argv[4], nullptr, 10));
    auto pick = [&](int n) { return (int)(rng() % (uint64_t)n); };
    char why[128] = "";

    // a*b + c: a multiply then an add, two ops the barrier keeps apart.
    {
        EltProgram p{};
        p.n = 1 << 20;
        p.cols = 1;
        for (int s = 0; s < 3; ++s) p.src[s] = (const float *)(uintptr_t)(0x1000000u * (s + 1));
        p.dst[0] = (float *)(uintptr_t)0x9000000u;
        auto ld = [](int r, int s) { EltInstr i{}; i.op = fg::kEltLoad; i.dst = r; i.a = s; return i; };
        EltInstr m{}, a{}, st{};
        m.op = fg::kEltMul, m.dst = 3, m.a = 0, m.b = 1;
        a.op = fg::kEltAdd, a.dst = 4, a.a = 3, a.b = 2;
        st.op = fg::kEltStore, st.a = 0, st.b = 4;
        for (EltInstr i : {ld(0, 0), ld(1, 1), ld(2, 2), m, a, st}) p.ins[p.n_instr++] = i;
        fg::EltJitShape s;
        s.quads = 4;
        s.src_al = s.dst_al = ~0u;
        const std::string src = fg::elt_jit_source(p, s, why, sizeof why);
        if (src.empty()) return printf("FAIL a*b+c: %s\n", why), 1;
        std::string nobar = src;
        for (size_t k; (k = nobar.find("fgj::bar(")) != std::string::npos;) nobar.replace(k, 9, "(");
        if (!compile(csrc, src, out + "/fma_bar.co") || !compile(csrc, nobar, out + "/fma_nobar.co"))
            return 1;
    }

    const uint8_t unaries[] = {fg::kEltNeg, fg::kEltRelu, fg::kEltGelu, fg::kEltElu,
                               fg::kEltTanh, fg::kEltExp, fg::kEltLog, fg::kEltAbs,
                               fg::kEltReluD, fg::kEltGeluD, fg::kEltEluD, fg::kEltSign,
                               fg::kEltRound};
    const uint8_t binaries[] = {fg::kEltAdd, fg::kEltSub, fg::kEltMul, fg::kEltDiv, fg::kEltMax};
    for (int t = 0; t < programs; ++t) {
        EltProgram p{};
        p.n = 1 + (uint64_t)pick(1 << 24);
        p.cols = 1 + (uint32_t)pick(5000);
        p.labels = (const uint32_t *)(uintptr_t)0x7000000u;
        // Sources 0..5 and destinations 0..3 at distinct addresses, but
        // destination 3 is source 5 (loads of it stay in program order).
        for (int s = 0; s < 6; ++s) p.src[s] = (const float *)(uintptr_t)(0x10000000ull * (s + 1));
        for (int d = 0; d < 3; ++d) p.dst[d] = (float *)(uintptr_t)(0x100000000ull * (d + 1));
        p.dst[3] = (float *)p.src[5];
        bool written[fg::kEltRegs] = {};
        int nw = 0;
        auto any_written = [&]() {
            int r;
            do r = pick(fg::kEltRegs); while (!written[r]);
            return r;
        };
        const int len = 2 + pick(30);
        for (int k = 0; k < len; ++k) {
            EltInstr in{};
            const int kind = nw == 0 ? 0 : pick(10);
            const int dst = pick(fg::kEltRegs);
            if (kind <= 2) {
                in.op = fg::kEltLoad;
                in.a = (uint8_t)pick(6);
                in.b = (uint8_t)pick(3);
                in.c = (uint8_t)(pick(6) < 4 ? fg::kModeFull : pick(2) ? fg::kModeRow : fg::kModeScalar);
            } else if (kind == 3) {
                in.op = pick(3) == 0 ? fg::kEltLabelEq : fg::kEltImm;
                in.imm = std::uniform_real_distribution<float>(-3.0f, 3.0f)(rng);
            } else if (kind <= 5) {
                in.op = pick(4) == 0 ? fg::kEltAccum : fg::kEltStore;
                in.a = (uint8_t)pick(4);
                in.b = (uint8_t)any_written();
                in.c = (uint8_t)pick(3);
                p.ins[p.n_instr++] = in;
                continue;
            } else if (kind <= 7) {
                in.op = unaries[pick(sizeof unaries)];
                in.a = (uint8_t)any_written();
                in.c = (uint8_t)pick(3);  // the element type of a round
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
        fg::EltJitShape s;
        s.quads = 1 << pick(3);
        s.nt = pick(2);
        s.src_al = (uint32_t)rng();
        s.dst_al = (uint32_t)rng();
        s.cols4 = pick(2);
        const std::string src = fg::elt_jit_source(p, s, why, sizeof why);
        if (src.empty()) return printf("FAIL program %d: %s\n", t, why), 1;
        if (!compile(csrc, src, out + "/k" + std::to_string(t) + ".co")) return 1;
    }
    printf("OK %d\n", programs);
    return 0;
}
