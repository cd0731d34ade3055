// fg_elt_jit.cpp -- elementwise programs compiled at run time: the kernel
// source of fg_elt_jit.h compiled with hipRTC for the context's device,
// loaded as a code object and kept for the life of the process, one kernel
// per (device, source).  The reference's ROCm backend compiles every fused
// kernel it generates the same way (GpuBackend::compile,
// crates/fused_gpu/src/dispatch/mod.rs:210; rocm/mod.rs:140-170: -O3, no
// fast math); here the interpreter of k_eltwise_prog.hip remains the path
// of small programs and of graph captures that meet a program not compiled
// yet.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "fg_elt_jit.h"
#include "fg_internal.h"

// kJitHeaders: {name, text} of the device headers a generated kernel
// includes (fg_half.h, fg_act.h, fg_elt_ops.h), written by the build from
// the sources beside this file.
#include "fg_jit_headers.inc"

namespace fg {
namespace {

// Programs over at least this many elements are compiled in the default
// mode: below it a launch costs more than the interpreter's scalar work.
constexpr uint64_t kJitMinElems = uint64_t(1) << 20;

struct JitKernel {
    hipModule_t module = nullptr;
    hipFunction_t fn = nullptr;
};

std::mutex g_mu;  // guards g_cache (compiles run under it: they are rare)
std::map<std::pair<int, std::string>, JitKernel> g_cache;
std::atomic<int> g_mode{-1};
std::atomic<uint64_t> g_compiled{0}, g_jit_launches{0}, g_interp_launches{0};

int mode() {
    int m = g_mode.load(std::memory_order_acquire);
    if (m >= 0) return m;
    const char *e = getenv("FG_ELTWISE_MODE");
    m = FG_ELTWISE_COMPILE_LARGE;
    if (e && e[0] >= '0' && e[0] <= '2' && e[1] == 0) m = e[0] - '0';
    int expect = -1;
    g_mode.compare_exchange_strong(expect, m, std::memory_order_acq_rel);
    return g_mode.load(std::memory_order_acquire);
}

bool aligned(const void *q, int dt) {
    return (((uintptr_t)q) & (dt == FG_DTYPE_F32 ? 15u : 7u)) == 0;
}

// hipRTC compile of one kernel source; fills `code`.
int compile(const std::string &src, std::vector<char> &code) {
    std::vector<const char *> names, texts;
    for (const auto &h : kJitHeaders) {
        names.push_back(h.name);
        texts.push_back(h.text);
    }
    names.push_back("fg_elt_jit_prelude.h");
    texts.push_back(elt_jit_prelude());
    hiprtcProgram prog = nullptr;
    hiprtcResult r = hiprtcCreateProgram(&prog, src.c_str(), "fg_elt_kernel.hip", (int)names.size(),
                                         texts.data(), names.data());
    FG_REQUIRE(r == HIPRTC_SUCCESS, FG_ERR_INTERNAL, "eltwise compile: hiprtcCreateProgram: %s",
               hiprtcGetErrorString(r));
    // The library's own device flags: gfx950, -O3, no packed-fp32 VALU
    // instructions (some of their forms gave silent wrong results on the
    // target machines), the compiler's default contraction within an op.
    const char *opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                          "-target-feature", "-Xclang", "-packed-fp32-ops"};
    r = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n + 1, '\0');
        if (n) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        set_error("eltwise compile: %s: %.1500s", hiprtcGetErrorString(r), log.c_str());
        return FG_ERR_INTERNAL;
    }
    size_t n = 0;
    r = hiprtcGetCodeSize(prog, &n);
    if (r == HIPRTC_SUCCESS) {
        code.resize(n);
        r = hiprtcGetCode(prog, code.data());
    }
    hiprtcDestroyProgram(&prog);
    FG_REQUIRE(r == HIPRTC_SUCCESS && !code.empty(), FG_ERR_INTERNAL,
               "eltwise compile: no code object (%s)", hiprtcGetErrorString(r));
    return FG_OK;
}

// The compiled kernel of `src` on the context's device: from the cache, or
// compiled and loaded now unless `may_build` is false (then fn stays NULL).
int kernel_for(fg_ctx *ctx, const std::string &src, bool may_build, hipFunction_t *fn) {
    *fn = nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    const auto key = std::make_pair(ctx->device, src);
    auto it = g_cache.find(key);
    if (it != g_cache.end()) {
        *fn = it->second.fn;
        return FG_OK;
    }
    if (!may_build) return FG_OK;
    std::vector<char> code;
    if (int rc = compile(src, code)) return rc;
    // FG_ELTWISE_DUMP=<directory>: each kernel's source and code object are
    // written there as it is compiled, fg_elt_<n>.hip / .co (the reference
    // logs its generated kernels under DebugCompilationOptions::
    // PRETTY_PRINT_IR, rocm/generate.rs:38-66).
    if (const char *dir = getenv("FG_ELTWISE_DUMP")) {
        const std::string stem = std::string(dir) + "/fg_elt_" +
                                 std::to_string(g_compiled.load(std::memory_order_relaxed));
        if (FILE *f = fopen((stem + ".hip").c_str(), "w")) {
            fwrite(src.data(), 1, src.size(), f);
            fclose(f);
        }
        if (FILE *f = fopen((stem + ".co").c_str(), "wb")) {
            fwrite(code.data(), 1, code.size(), f);
            fclose(f);
        }
    }
    JitKernel k;
    FG_HIP(hipSetDevice(ctx->device));
    FG_HIP(hipModuleLoadData(&k.module, code.data()));
    const hipError_t e = hipModuleGetFunction(&k.fn, k.module, kEltJitKernel);
    if (e != hipSuccess) {
        (void)hipModuleUnload(k.module);
        return hip_fail(e, "hipModuleGetFunction", __FILE__, __LINE__);
    }
    g_cache.emplace(key, k);
    g_compiled.fetch_add(1, std::memory_order_relaxed);
    *fn = k.fn;
    return FG_OK;
}

}  // namespace

bool eltwise_jit_selected(const EltProgram &p) {
    const int m = mode();
    return m == FG_ELTWISE_COMPILE_ALL || (m == FG_ELTWISE_COMPILE_LARGE && p.n >= kJitMinElems);
}

void eltwise_count_interpreted() { g_interp_launches.fetch_add(1, std::memory_order_relaxed); }

// A validated program with `live` values at most live at once: its kernel
// source, compiled and loaded when missing (never during a stream capture,
// whose graph would then hold a launch of a module loaded inside it), and
// launched unless `prepare_only`.  *launched reports whether it ran here.
int eltwise_jit(fg_ctx *ctx, const EltProgram &p, int live, bool prepare_only, bool *launched) {
    *launched = false;
    EltJitShape s;
    s.quads = elt_jit_quads(live);
    s.nt = p.n >= (uint64_t(1) << 22);  // as the interpreter: streaming past the L2 caches
    s.cols4 = p.cols % 4 == 0;
    // A pointer takes quad accesses when every access of the program allows
    // them (a source read as two element types: aligned for both).
    s.src_al = s.dst_al = ~0u;
    for (int k = 0; k < p.n_instr; ++k) {
        const EltInstr &in = p.ins[k];
        if (in.op == kEltLoad && !aligned(p.src[in.a], in.b)) s.src_al &= ~(1u << in.a);
        if ((in.op == kEltStore || in.op == kEltAccum) && !aligned(p.dst[in.a], in.c))
            s.dst_al &= ~(1u << in.a);
    }
    char why[128] = "";
    const std::string src = elt_jit_source(p, s, why, sizeof why);
    FG_REQUIRE(!src.empty(), FG_ERR_INTERNAL, "eltwise compile: %s", why);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    FG_HIP(hipStreamIsCapturing(ctx->stream, &cap));
    hipFunction_t fn = nullptr;
    if (int rc = kernel_for(ctx, src, cap == hipStreamCaptureStatusNone, &fn)) return rc;
    if (!fn || prepare_only) return FG_OK;
    EltJitArgs a;
    memset(&a, 0, sizeof a);
    for (int k = 0; k < kEltMaxSrc; ++k) a.src[k] = p.src[k];
    for (int k = 0; k < kEltMaxDst; ++k) a.dst[k] = p.dst[k];
    a.labels = p.labels;
    a.n = p.n;
    a.cols = p.cols;
    // One pass per workgroup where the grid allows it, within 32-bit grid
    // arithmetic (the pass loop covers the rest).
    const uint64_t span = 256ull * (uint64_t)s.quads;
    uint64_t blocks = ((p.n + 3) / 4 + span - 1) / span;
    constexpr uint64_t kMaxBlocks = (uint64_t(1) << 32) / 256 / 2;
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    void *params[] = {&a};
    FG_HIP(hipModuleLaunchKernel(fn, (unsigned)blocks, 1, 1, 256, 1, 1, 0, ctx->stream, params,
                                 nullptr));
    g_jit_launches.fetch_add(1, std::memory_order_relaxed);
    *launched = true;
    return FG_OK;
}

}  // namespace fg

FG_API int fg_eltwise_set_mode(int mode, int *previous) {
    FG_REQUIRE(mode >= FG_ELTWISE_INTERPRET && mode <= FG_ELTWISE_COMPILE_ALL,
               FG_ERR_INVALID_ARGUMENT, "fg_eltwise_set_mode: bad mode %d", mode);
    const int prev = fg::mode();
    fg::g_mode.store(mode, std::memory_order_release);
    if (previous) *previous = prev;
    return FG_OK;
}

FG_API int fg_eltwise_stats(uint64_t *kernels_compiled, uint64_t *compiled_launches,
                            uint64_t *interpreted_launches) {
    if (kernels_compiled) *kernels_compiled = fg::g_compiled.load(std::memory_order_relaxed);
    if (compiled_launches) *compiled_launches = fg::g_jit_launches.load(std::memory_order_relaxed);
    if (interpreted_launches)
        *interpreted_launches = fg::g_interp_launches.load(std::memory_order_relaxed);
    return FG_OK;
}
