// k_noalloc.hip -- fg_bias_grad_noalloc: the bias-gradient column reduction
// (fg_bias_grad's kernels, fg_bias_grad.h) for callers that cannot allocate
// device memory: code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc.  Its partial sums live in `scratch`, a fixed device
// array of this library (each GPU holds its own copy until the process
// ends), instead of the context workspace that fg_bias_grad grows on demand.
//
// Host code never passes `scratch` itself to a kernel: in host code that name
// is a host-side stand-in, not a device address.  fg_ctx_create calls
// noalloc_init() once per device, with the device current, which looks up the
// device address with hipGetSymbolAddress and keeps it per device.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU
// (two streams, two host threads) race on it and must be ordered by the
// caller.  Nothing in the array needs to start at zero: the first pass writes
// every partial sum the second pass reads.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "fg_bias_grad.h"
#include "fg_internal.h"

namespace {

// 4 MiB: the partial sums of any N <= 1,048,576 columns at the split count
// fg_bias_grad uses (splits * N stays <= 2^20 for every such N), so the two
// entry points run the same launches and give the same bits.
constexpr uint64_t kScratchFloats = uint64_t(1) << 20;
__device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
// Device address of `scratch`, per device.  Written once under the mutex by
// noalloc_init; read without it by fg_bias_grad_noalloc on any host thread,
// so each entry is atomic (release store, acquire load).
std::atomic<float *> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

}  // namespace

namespace fg {

// Looks up this device's copy of `scratch` (once per device).  The caller
// has made `device` current.
int noalloc_init(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    FG_REQUIRE(device >= 0 && device < kMaxDevices, FG_ERR_UNSUPPORTED,
               "noalloc_init: device %d beyond the %d devices this library tracks", device,
               kMaxDevices);
    if (g_scratch_ptr[device].load(std::memory_order_acquire)) return FG_OK;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
        return hip_fail(e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
    FG_REQUIRE(ptr, FG_ERR_INTERNAL, "noalloc_init: no device address for scratch");
    g_scratch_ptr[device].store(static_cast<float *>(ptr), std::memory_order_release);
    return FG_OK;
}

}  // namespace fg

FG_API int fg_bias_grad_noalloc(fg_ctx *ctx, int dtype, int M, int N, const void *d_dZ, int ld,
                                void *d_dbias, int accumulate) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "fg_bias_grad_noalloc: ctx is NULL");
    FG_REQUIRE(dtype >= FG_DTYPE_F32 && dtype <= FG_DTYPE_BF16, FG_ERR_INVALID_ARGUMENT,
               "fg_bias_grad_noalloc: bad dtype %d", dtype);
    FG_REQUIRE(M >= 0 && N >= 0 && ld >= N, FG_ERR_SHAPE,
               "fg_bias_grad_noalloc: bad shape M=%d N=%d ld=%d", M, N, ld);
    if (N == 0) return FG_OK;
    FG_REQUIRE(d_dZ && d_dbias, FG_ERR_INVALID_ARGUMENT, "fg_bias_grad_noalloc: NULL pointer");
    const fg::colsum::Split sp =
        fg::colsum::split_of(ctx->cu_count > 0 ? ctx->cu_count : 256, M, N);
    FG_REQUIRE(sp.partial_floats(N) <= kScratchFloats, FG_ERR_OUT_OF_BOUNDS,
               "fg_bias_grad_noalloc: %d columns need %llu bytes of partial sums; the "
               "fixed scratch holds %llu (N <= %llu)",
               N, (unsigned long long)(sp.partial_floats(N) * sizeof(float)),
               (unsigned long long)(kScratchFloats * sizeof(float)),
               (unsigned long long)kScratchFloats);
    FG_REQUIRE(ctx->device >= 0 && ctx->device < kMaxDevices, FG_ERR_INTERNAL,
               "fg_bias_grad_noalloc: device %d beyond the tracked devices", ctx->device);
    float *partial = g_scratch_ptr[ctx->device].load(std::memory_order_acquire);
    FG_REQUIRE(partial, FG_ERR_INTERNAL, "fg_bias_grad_noalloc: scratch of device %d not set up",
               ctx->device);
    FG_HIP(hipSetDevice(ctx->device));
    FG_HIP(fg::colsum::launch(ctx->stream, sp, dtype, M, N, d_dZ, ld, d_dbias, accumulate,
                              partial));
    return FG_OK;
}
