// k_elementwise.hip -- HBM-bound elementwise kernels: activation backward,
// u32 fill, and the counter-based synthetic-data generator (host and device
// variants produce the same values for the same key).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "fg_act.h"
#include "fg_internal.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

// dZ = dH * act'(Z); unary backward of crates/ferrograd-nn/src/op/unary.rs.
__global__ __launch_bounds__(kThreads) void act_bwd_kernel(int act, uint64_t n,
                                                           const float *__restrict__ dH,
                                                           const float *__restrict__ Z,
                                                           float *__restrict__ dZ, int vec) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    if (vec) {
        const uint64_t n4 = n / 4;
        for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
            const f32x4 h = reinterpret_cast<const f32x4 *>(dH)[i];
            const f32x4 z = reinterpret_cast<const f32x4 *>(Z)[i];
            f32x4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = h[e] * fg::act_grad(act, z[e]);
            reinterpret_cast<f32x4 *>(dZ)[i] = r;
        }
        for (uint64_t i = n4 * 4 + (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
            dZ[i] = dH[i] * fg::act_grad(act, Z[i]);
    } else {
        for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
            dZ[i] = dH[i] * fg::act_grad(act, Z[i]);
    }
}

__global__ __launch_bounds__(kThreads) void fill_u32_kernel(uint32_t *__restrict__ dst,
                                                            uint32_t value, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        dst[i] = value;
}

// ---------------------------------------------------------------- RNG
__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 27;
    z *= 0x94D049BB133111EBull;
    z ^= z >> 31;
    return z;
}
__host__ __device__ inline uint64_t rng_key(uint64_t seed, uint64_t tensor_id) {
    return mix64(seed ^ mix64(tensor_id + 0x632BE59BD9B4E019ull));
}
__host__ __device__ inline uint64_t rng_draw(uint64_t key, uint64_t i) {
    return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}
__host__ __device__ inline float rng_uniform(uint64_t key, uint64_t i, float lo, float hi) {
    const double u = (double)(rng_draw(key, i) >> 40) * (1.0 / 16777216.0);
    return (float)((double)lo + ((double)hi - (double)lo) * u);
}
__host__ __device__ inline float rng_normal(uint64_t key, uint64_t i, float mean, float std) {
    const double u1 = (double)((rng_draw(key, 2 * i) >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(rng_draw(key, 2 * i + 1) >> 11) * (1.0 / 9007199254740992.0);
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    return (float)((double)mean + (double)std * z);
}
__host__ __device__ inline uint32_t rng_int(uint64_t key, uint64_t i, uint32_t bound) {
    return (uint32_t)(((rng_draw(key, i) >> 32) * (uint64_t)bound) >> 32);
}

__global__ __launch_bounds__(kThreads) void rng_kernel(int kind, uint64_t key, float a, float b,
                                                       uint32_t bound, void *dst, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        if (kind == 0)
            reinterpret_cast<float *>(dst)[i] = rng_uniform(key, i, a, b);
        else if (kind == 1)
            reinterpret_cast<float *>(dst)[i] = rng_normal(key, i, a, b);
        else
            reinterpret_cast<uint32_t *>(dst)[i] = rng_int(key, i, bound);
    }
}

// Host-side parallel loop over [0, n) on hardware threads.
template <class F>
void host_parallel_for(uint64_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (n < (1u << 16) || nt == 1) {
        for (uint64_t i = 0; i < n; ++i) f(i);
        return;
    }
    if (nt > 64) nt = 64;
    std::vector<std::thread> pool;
    const uint64_t per = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const uint64_t b = t * per, e = (b + per < n) ? b + per : n;
        if (b >= e) break;
        pool.emplace_back([=] {
            for (uint64_t i = b; i < e; ++i) f(i);
        });
    }
    for (auto &th : pool) th.join();
}

unsigned grid_for(uint64_t n, int cu_count) {
    uint64_t blocks = (n + kThreads - 1) / kThreads;
    const uint64_t cap = (uint64_t)(cu_count > 0 ? cu_count : 256) * 16;
    if (blocks > cap) blocks = cap;
    return blocks ? (unsigned)blocks : 1u;
}

int rng_dev(fg_ctx *ctx, int kind, uint64_t seed, uint64_t tid, float a, float b,
            uint32_t bound, void *dst, uint64_t n) {
    FG_REQUIRE(ctx && (dst || !n), FG_ERR_INVALID_ARGUMENT, "fg_rng_*_dev: NULL argument");
    if (!n) return FG_OK;
    FG_HIP(hipSetDevice(ctx->device));
    rng_kernel<<<grid_for(n, ctx->cu_count), kThreads, 0, ctx->stream>>>(
        kind, rng_key(seed, tid), a, b, bound, dst, n);
    FG_LAUNCH_CHECK("rng_kernel");
    return FG_OK;
}

}  // namespace

FG_API int fg_act_bwd_f32(fg_ctx *ctx, int act, uint64_t n, const float *d_dH, const float *d_Z,
                          float *d_dZ) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "fg_act_bwd_f32: ctx is NULL");
    FG_REQUIRE(act >= 0 && act <= 2, FG_ERR_INVALID_ARGUMENT, "fg_act_bwd_f32: bad act %d", act);
    if (!n) return FG_OK;
    FG_REQUIRE(d_dH && d_Z && d_dZ, FG_ERR_INVALID_ARGUMENT, "fg_act_bwd_f32: NULL pointer");
    FG_HIP(hipSetDevice(ctx->device));
    const int vec = ((((uintptr_t)d_dH) | ((uintptr_t)d_Z) | ((uintptr_t)d_dZ)) & 15u) == 0;
    // One 16-byte quad per thread and as many workgroups as that takes (a
    // plain stream, each workgroup touching one contiguous 16 KiB span),
    // up to the grid limit; the kernel's loop covers anything beyond.
    const uint64_t items = vec ? (n + 3) / 4 : n;
    const unsigned grid =
        (unsigned)std::min<uint64_t>((items + kThreads - 1) / kThreads, 1u << 30);
    act_bwd_kernel<<<grid, kThreads, 0, ctx->stream>>>(act, n, d_dH, d_Z, d_dZ, vec);
    FG_LAUNCH_CHECK("act_bwd_kernel");
    return FG_OK;
}

FG_API int fg_fill_u32(fg_ctx *ctx, void *d_dst, uint32_t value, uint64_t count) {
    FG_REQUIRE(ctx && (d_dst || !count), FG_ERR_INVALID_ARGUMENT, "fg_fill_u32: NULL argument");
    if (!count) return FG_OK;
    FG_HIP(hipSetDevice(ctx->device));
    fill_u32_kernel<<<grid_for(count, ctx->cu_count), kThreads, 0, ctx->stream>>>(
        (uint32_t *)d_dst, value, count);
    FG_LAUNCH_CHECK("fill_u32_kernel");
    return FG_OK;
}

FG_API int fg_rng_uniform_host(uint64_t seed, uint64_t tensor_id, float lo, float hi, float *dst,
                               uint64_t n) {
    FG_REQUIRE(dst || !n, FG_ERR_INVALID_ARGUMENT, "fg_rng_uniform_host: dst is NULL");
    const uint64_t key = rng_key(seed, tensor_id);
    host_parallel_for(n, [=](uint64_t i) { dst[i] = rng_uniform(key, i, lo, hi); });
    return FG_OK;
}

FG_API int fg_rng_normal_host(uint64_t seed, uint64_t tensor_id, float mean, float std, float *dst,
                              uint64_t n) {
    FG_REQUIRE(dst || !n, FG_ERR_INVALID_ARGUMENT, "fg_rng_normal_host: dst is NULL");
    const uint64_t key = rng_key(seed, tensor_id);
    host_parallel_for(n, [=](uint64_t i) { dst[i] = rng_normal(key, i, mean, std); });
    return FG_OK;
}

FG_API int fg_rng_int_host(uint64_t seed, uint64_t tensor_id, uint32_t bound, uint32_t *dst,
                           uint64_t n) {
    FG_REQUIRE(dst || !n, FG_ERR_INVALID_ARGUMENT, "fg_rng_int_host: dst is NULL");
    FG_REQUIRE(bound > 0, FG_ERR_INVALID_ARGUMENT, "fg_rng_int_host: bound must be > 0");
    const uint64_t key = rng_key(seed, tensor_id);
    host_parallel_for(n, [=](uint64_t i) { dst[i] = rng_int(key, i, bound); });
    return FG_OK;
}

FG_API int fg_rng_uniform_dev(fg_ctx *ctx, uint64_t seed, uint64_t tensor_id, float lo, float hi,
                              float *d_dst, uint64_t n) {
    return rng_dev(ctx, 0, seed, tensor_id, lo, hi, 0, d_dst, n);
}

FG_API int fg_rng_normal_dev(fg_ctx *ctx, uint64_t seed, uint64_t tensor_id, float mean,
                             float std, float *d_dst, uint64_t n) {
    return rng_dev(ctx, 1, seed, tensor_id, mean, std, 0, d_dst, n);
}

FG_API int fg_rng_int_dev(fg_ctx *ctx, uint64_t seed, uint64_t tensor_id, uint32_t bound,
                          uint32_t *d_dst, uint64_t n) {
    FG_REQUIRE(bound > 0, FG_ERR_INVALID_ARGUMENT, "fg_rng_int_dev: bound must be > 0");
    return rng_dev(ctx, 2, seed, tensor_id, 0.f, 0.f, bound, d_dst, n);
}
