// fg_runtime.cpp -- context, buffers, errors: the launch-layer half of the
// backend.  Replaces rocm::GpuContext (crates/fused_gpu/src/dispatch/backend/
// rocm/mod.rs:57-429) and the buffer half of the GpuBackend trait
// (crates/fused_gpu/src/dispatch/mod.rs:147-261).  Code objects are compiled
// ahead of time for gfx950 and linked into this library; there is no runtime
// compilation (the reference compiles generated source with hipRTC,
// rocm/mod.rs:140-170).
#include <cstdarg>
#include <cstring>

#include "fg_internal.h"

namespace fg {

static thread_local std::string g_last_error;

void set_error(const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int hip_fail(hipError_t e, const char *what, const char *file, int line) {
    set_error("%s failed: %s (%s:%d)", what, hipGetErrorString(e), file, line);
    switch (e) {
        case hipErrorOutOfMemory: return FG_ERR_OUT_OF_MEMORY;
        case hipErrorNoDevice: return FG_ERR_NO_DEVICE;
        case hipErrorInvalidValue:
        case hipErrorInvalidDevice:
        case hipErrorInvalidDevicePointer: return FG_ERR_INVALID_ARGUMENT;
        case hipErrorNotSupported: return FG_ERR_UNSUPPORTED;
        default: return FG_ERR_DEVICE;
    }
}

void *workspace(fg_ctx *ctx, uint64_t bytes) {
    if (bytes <= ctx->ws_bytes) return ctx->ws;
    if (ctx->ws_fixed) {
        set_error("workspace: %llu bytes requested from a fixed workspace of %llu bytes",
                  (unsigned long long)bytes, (unsigned long long)ctx->ws_bytes);
        return nullptr;
    }
    // Grow geometrically (at least double, rounded up to 1 MiB): every
    // replaced buffer is kept until the context is destroyed (below), so
    // the kept buffers total at most about twice the final size however the
    // requests creep upward.
    uint64_t want = (bytes + (1u << 20) - 1) & ~uint64_t((1u << 20) - 1);
    if (want < 2 * ctx->ws_bytes) want = 2 * ctx->ws_bytes;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        set_error("workspace: hipMalloc(%llu) failed: %s", (unsigned long long)want,
                  hipGetErrorString(e));
        return nullptr;
    }
    // The old workspace may be baked into a captured graph or still in use
    // by queued work: keep it until the context is destroyed.
    if (ctx->ws) ctx->ws_retired.push_back(ctx->ws);
    ctx->ws = p;
    ctx->ws_bytes = want;
    return p;
}

}  // namespace fg

FG_API const char *fg_last_error_msg(void) { return fg::g_last_error.c_str(); }

FG_API int fg_version(void) { return 100; }

FG_API int fg_ctx_create(int device, void *stream, fg_ctx **out) {
    FG_REQUIRE(out, FG_ERR_INVALID_ARGUMENT, "fg_ctx_create: out is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        fg::set_error("fg_ctx_create: no HIP device (%s)", hipGetErrorString(e));
        return FG_ERR_NO_DEVICE;
    }
    FG_REQUIRE(device >= 0 && device < n, FG_ERR_INVALID_ARGUMENT,
               "fg_ctx_create: device %d out of range (%d devices)", device, n);
    FG_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    FG_HIP(hipGetDeviceProperties(&prop, device));
    fg_ctx *ctx = new fg_ctx;
    ctx->device = device;
    ctx->cu_count = prop.multiProcessorCount;
    snprintf(ctx->arch, sizeof ctx->arch, "%s", prop.gcnArchName);
    // The arch string carries feature suffixes ("gfx950:sramecc+:xnack-").
    if (char *colon = strchr(ctx->arch, ':')) *colon = 0;
    if (strcmp(ctx->arch, "gfx950") != 0) {
        fg::set_error("fg_ctx_create: device %d is %s; this library carries gfx950 code only",
                      device, ctx->arch);
        delete ctx;
        return FG_ERR_UNSUPPORTED;
    }
    // Device address of the fixed scratch of fg_bias_grad_noalloc.
    if (int rc = fg::noalloc_init(device)) {
        delete ctx;
        return rc;
    }
    if (stream) {
        ctx->stream = (hipStream_t)stream;
        ctx->own_stream = false;
    } else {
        hipError_t se = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
        if (se != hipSuccess) {
            delete ctx;
            return fg::hip_fail(se, "hipStreamCreateWithFlags", __FILE__, __LINE__);
        }
        ctx->own_stream = true;
    }
    *out = ctx;
    return FG_OK;
}

FG_API int fg_ctx_destroy(fg_ctx *ctx) {
    if (!ctx) return FG_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    for (void *w : ctx->ws_retired) (void)hipFree(w);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return FG_OK;
}

FG_API int fg_ctx_target(fg_ctx *ctx, char *arch, size_t arch_len, uint32_t *flags,
                         int *cu_count) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "fg_ctx_target: ctx is NULL");
    if (arch && arch_len) snprintf(arch, arch_len, "%s", ctx->arch);
    if (flags) *flags = FG_TARGET_LIN_ACC;
    if (cu_count) *cu_count = ctx->cu_count;
    return FG_OK;
}

FG_API int fg_ctx_stream(fg_ctx *ctx, void **stream) {
    FG_REQUIRE(ctx && stream, FG_ERR_INVALID_ARGUMENT, "fg_ctx_stream: NULL argument");
    *stream = (void *)ctx->stream;
    return FG_OK;
}

FG_API int fg_ctx_reserve_workspace(fg_ctx *ctx, uint64_t bytes) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "fg_ctx_reserve_workspace: ctx is NULL");
    FG_HIP(hipSetDevice(ctx->device));
    if (!fg::workspace(ctx, bytes)) return FG_ERR_OUT_OF_MEMORY;
    return FG_OK;
}

FG_API int fg_sync(fg_ctx *ctx) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "fg_sync: ctx is NULL");
    FG_HIP(hipStreamSynchronize(ctx->stream));
    return FG_OK;
}

FG_API int fg_is_ready(fg_ctx *ctx, int *ready) {
    FG_REQUIRE(ctx && ready, FG_ERR_INVALID_ARGUMENT, "fg_is_ready: NULL argument");
    hipError_t e = hipStreamQuery(ctx->stream);
    if (e == hipSuccess) {
        *ready = 1;
        return FG_OK;
    }
    if (e == hipErrorNotReady) {
        *ready = 0;
        return FG_OK;
    }
    return fg::hip_fail(e, "hipStreamQuery", __FILE__, __LINE__);
}

// ------------------------------------------------------------------ buffers
static int buf_new(fg_ctx *ctx, uint64_t bytes, fg_buf **out) {
    FG_REQUIRE(ctx && out, FG_ERR_INVALID_ARGUMENT, "fg_buf_alloc: NULL argument");
    FG_HIP(hipSetDevice(ctx->device));
    fg_buf *b = new fg_buf;
    b->device = ctx->device;
    b->bytes = bytes;
    if (bytes) {
        hipError_t e = hipMalloc(&b->ptr, bytes);
        if (e != hipSuccess) {
            delete b;
            return fg::hip_fail(e, "hipMalloc", __FILE__, __LINE__);
        }
    }
    *out = b;
    return FG_OK;
}

FG_API int fg_buf_alloc(fg_ctx *ctx, uint64_t bytes, fg_buf **out) {
    return buf_new(ctx, bytes, out);
}

FG_API int fg_buf_alloc_zeroed(fg_ctx *ctx, uint64_t bytes, fg_buf **out) {
    int rc = buf_new(ctx, bytes, out);
    if (rc) return rc;
    if (bytes) {
        FG_HIP(hipMemsetAsync((*out)->ptr, 0, bytes, ctx->stream));
        FG_HIP(hipStreamSynchronize(ctx->stream));
    }
    return FG_OK;
}

FG_API int fg_buf_alloc_init(fg_ctx *ctx, const void *src, uint64_t bytes, fg_buf **out) {
    FG_REQUIRE(src || !bytes, FG_ERR_INVALID_ARGUMENT, "fg_buf_alloc_init: src is NULL");
    int rc = buf_new(ctx, bytes, out);
    if (rc) return rc;
    if (bytes) {
        FG_HIP(hipMemcpyAsync((*out)->ptr, src, bytes, hipMemcpyHostToDevice, ctx->stream));
        FG_HIP(hipStreamSynchronize(ctx->stream));
    }
    return FG_OK;
}

FG_API int fg_buf_free(fg_buf *buf) {
    if (!buf) return FG_OK;
    if (buf->ptr) {
        // hipFree waits for outstanding work on the device; the context that
        // allocated the buffer may already be destroyed.
        (void)hipSetDevice(buf->device);
        hipError_t e = hipFree(buf->ptr);
        if (e != hipSuccess) {
            delete buf;
            return fg::hip_fail(e, "hipFree", __FILE__, __LINE__);
        }
    }
    delete buf;
    return FG_OK;
}

FG_API uint64_t fg_buf_size_bytes(const fg_buf *buf) { return buf ? buf->bytes : 0; }

FG_API void *fg_buf_device_ptr(const fg_buf *buf) { return buf ? buf->ptr : nullptr; }

FG_API int fg_upload(fg_ctx *ctx, fg_buf *dst, const void *src, uint64_t bytes,
                     uint64_t dst_off) {
    FG_REQUIRE(ctx && dst && (src || !bytes), FG_ERR_INVALID_ARGUMENT,
               "fg_upload: NULL argument");
    FG_REQUIRE(dst_off <= dst->bytes && bytes <= dst->bytes - dst_off, FG_ERR_OUT_OF_BOUNDS,
               "fg_upload: %llu bytes at offset %llu exceed buffer of %llu bytes",
               (unsigned long long)bytes, (unsigned long long)dst_off,
               (unsigned long long)dst->bytes);
    if (!bytes) return FG_OK;
    FG_HIP(hipMemcpyAsync((char *)dst->ptr + dst_off, src, bytes, hipMemcpyHostToDevice,
                          ctx->stream));
    FG_HIP(hipStreamSynchronize(ctx->stream));
    return FG_OK;
}

FG_API int fg_download(fg_ctx *ctx, const fg_buf *src, void *dst, uint64_t bytes,
                       uint64_t src_off) {
    FG_REQUIRE(ctx && src && (dst || !bytes), FG_ERR_INVALID_ARGUMENT,
               "fg_download: NULL argument");
    FG_REQUIRE(src_off <= src->bytes && bytes <= src->bytes - src_off, FG_ERR_OUT_OF_BOUNDS,
               "fg_download: %llu bytes at offset %llu exceed buffer of %llu bytes",
               (unsigned long long)bytes, (unsigned long long)src_off,
               (unsigned long long)src->bytes);
    if (!bytes) return FG_OK;
    FG_HIP(hipMemcpyAsync(dst, (const char *)src->ptr + src_off, bytes, hipMemcpyDeviceToHost,
                          ctx->stream));
    FG_HIP(hipStreamSynchronize(ctx->stream));
    return FG_OK;
}

FG_API int fg_copy(fg_ctx *ctx, const fg_buf *src, fg_buf *dst) {
    FG_REQUIRE(ctx && src && dst, FG_ERR_INVALID_ARGUMENT, "fg_copy: NULL argument");
    FG_REQUIRE(src->bytes <= dst->bytes, FG_ERR_OUT_OF_BOUNDS,
               "fg_copy: source (%llu bytes) larger than destination (%llu bytes)",
               (unsigned long long)src->bytes, (unsigned long long)dst->bytes);
    if (!src->bytes) return FG_OK;
    FG_HIP(hipMemcpyAsync(dst->ptr, src->ptr, src->bytes, hipMemcpyDeviceToDevice,
                          ctx->stream));
    return FG_OK;
}
