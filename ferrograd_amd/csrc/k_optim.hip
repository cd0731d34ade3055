// k_optim.hip -- multi-tensor SGD and Adam for gfx950.
//
// One launch updates a whole tensor list.  The reference instead captures
// one optimiser kernel per input tensor into a hipGraph
// (crates/fused_gpu/src/dispatch/backend/kernel/optim.rs:12-158,
// rocm/mod.rs:268-322) and sizes every launch from the root node's shape
// (optim.rs:13-25), which is wrong for weights of other shapes.
//
// Work decomposition: each tensor is cut into chunks of CHUNK elements; a
// device-resident chunk table maps blockIdx.x -> (tensor, first element), so
// one launch covers tensors of any sizes and the table is built once per
// list (the per-step scalars travel as kernel arguments, which keeps the
// launch capturable in a hipGraph).  Every element is touched by exactly one
// thread: streams are read once and written once (Adam: 16 B read + 12 B
// written per parameter; SGD: 8 B read + 4-8 B written), with 16-byte
// non-temporal accesses -- the kernels are HBM-bound.
//
// This unit is compiled with -ffp-contract=off and uses only correctly
// rounded operations, so each element goes through exactly the fp32
// operation sequence of the CPU restatement (bit-exact parity).
#include <hip/hip_runtime.h>

#include <cmath>
#include <vector>

#include "fg_optim.h"

namespace {

using namespace fg::optim;

// m = b1*m + (1-b1)*g ; v = b2*v + (1-b2)*(g*g) ;
// p = p - (step_size*m) / (sqrt(v)*inv_sqrt_bc2 + eps)
// Plain operators: this unit is compiled without contraction, and HIP's
// sqrtf and '/' are correctly rounded (the __fsqrt_rn intrinsic is not: it
// maps to the hardware approximation).
__device__ inline void adam_elem(float &p, float g, float &m, float &v, float b1,
                                 float omb1, float b2, float omb2, float eps,
                                 float step_size, float inv_sqrt_bc2) {
    const float mi = b1 * m + omb1 * g;
    const float vi = b2 * v + omb2 * (g * g);
    const float denom = sqrtf(vi) * inv_sqrt_bc2 + eps;
    p = p - (step_size * mi) / denom;
    m = mi;
    v = vi;
}

// One chunk of a 16-bit tensor: the update in fp32 (m, v stay fp32), the
// parameter rounded once to its type; the gradient read as stored.
__device__ void adam_chunk_h16(const MTTensor &t, uint64_t start, uint64_t end, float b1,
                               float b2, float eps, float step_size, float inv_sqrt_bc2,
                               int zero_grad) {
    uint16_t *p16 = reinterpret_cast<uint16_t *>(t.p);
    uint16_t *g16 = reinterpret_cast<uint16_t *>(t.g);
    const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
    for (uint64_t i = start + threadIdx.x; i < end; i += kThreads) {
        float p = fg::h16_to_f(t.dtype, p16[i]), m = t.m[i], v = t.v[i];
        adam_elem(p, fg::h16_to_f(t.dtype, g16[i]), m, v, b1, omb1, b2, omb2, eps, step_size,
                  inv_sqrt_bc2);
        p16[i] = fg::f_to_h16(t.dtype, p);
        t.m[i] = m;
        t.v[i] = v;
        if (zero_grad) g16[i] = 0;
    }
}

__global__ __launch_bounds__(kThreads) void adam_mt_kernel(
    const MTTensor *__restrict__ tensors, const MTChunk *__restrict__ chunks, float b1,
    float b2, float eps, float step_size, float inv_sqrt_bc2, int zero_grad, int vec) {
    const MTChunk c = chunks[blockIdx.x];
    const MTTensor t = tensors[c.tensor];
    const uint64_t end = (c.start + kChunk < t.n) ? c.start + kChunk : t.n;
    if (t.dtype != fg::kF32) {
        adam_chunk_h16(t, c.start, end, b1, b2, eps, step_size, inv_sqrt_bc2, zero_grad);
        return;
    }
    const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
    if (vec) {
        f32x4 P[kUnroll], G[kUnroll], M[kUnroll], V[kUnroll];
        uint64_t idx[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            idx[u] = c.start + (uint64_t)(u * kThreads + threadIdx.x) * 4;
            if (idx[u] + 4 <= end) {
                P[u] = ld_nt(t.p + idx[u]);
                G[u] = ld_nt(t.g + idx[u]);
                M[u] = ld_nt(t.m + idx[u]);
                V[u] = ld_nt(t.v + idx[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (idx[u] + 4 <= end) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float pe = P[u][e], me = M[u][e], ve = V[u][e];
                    adam_elem(pe, G[u][e], me, ve, b1, omb1, b2, omb2, eps, step_size,
                              inv_sqrt_bc2);
                    P[u][e] = pe;
                    M[u][e] = me;
                    V[u][e] = ve;
                }
                st_nt(t.p + idx[u], P[u]);
                st_nt(t.m + idx[u], M[u]);
                st_nt(t.v + idx[u], V[u]);
                if (zero_grad) st_nt(t.g + idx[u], f32x4{0.f, 0.f, 0.f, 0.f});
            } else {
                for (uint64_t i = idx[u]; i < end && i < idx[u] + 4; ++i) {
                    float p = t.p[i], m = t.m[i], v = t.v[i];
                    adam_elem(p, t.g[i], m, v, b1, omb1, b2, omb2, eps, step_size,
                              inv_sqrt_bc2);
                    t.p[i] = p;
                    t.m[i] = m;
                    t.v[i] = v;
                    if (zero_grad) t.g[i] = 0.0f;
                }
            }
        }
    } else {
        for (uint64_t i = c.start + threadIdx.x; i < end; i += kThreads) {
            float p = t.p[i], m = t.m[i], v = t.v[i];
            adam_elem(p, t.g[i], m, v, b1, omb1, b2, omb2, eps, step_size, inv_sqrt_bc2);
            t.p[i] = p;
            t.m[i] = m;
            t.v[i] = v;
            if (zero_grad) t.g[i] = 0.0f;
        }
    }
}

// Adam with its per-step scalars in device memory: a one-thread kernel
// advances the step counter and derives step_size / inv_sqrt_bc2 (in
// double, rounded once to fp32) so that a captured hipGraph replays correct
// bias corrections on every step without host involvement.
struct AdamDevState {
    uint32_t step;
    float step_size;
    float inv_sqrt_bc2;
    float pad;
};

__global__ void adam_advance_kernel(AdamDevState *st, double lr, double b1, double b2) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const uint32_t t = st->step + 1;
    st->step = t;
    const double bc1 = 1.0 - pow(b1, (double)t);
    const double bc2 = 1.0 - pow(b2, (double)t);
    st->step_size = (float)(lr / bc1);
    st->inv_sqrt_bc2 = (float)(1.0 / sqrt(bc2));
}

// One chunk of the multi-tensor Adam update with the step's scalars.
__device__ __forceinline__ void adam_dev_chunk(const MTTensor *__restrict__ tensors,
                                               const MTChunk *__restrict__ chunks, uint32_t ci,
                                               float b1, float b2, float eps, float step_size,
                                               float inv_sqrt_bc2, int zero_grad, int vec) {
    const MTChunk c = chunks[ci];
    const MTTensor t = tensors[c.tensor];
    const uint64_t end = (c.start + kChunk < t.n) ? c.start + kChunk : t.n;
    if (t.dtype != fg::kF32) {
        adam_chunk_h16(t, c.start, end, b1, b2, eps, step_size, inv_sqrt_bc2, zero_grad);
        return;
    }
    const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
    if (vec) {
        f32x4 P[kUnroll], G[kUnroll], M[kUnroll], V[kUnroll];
        uint64_t idx[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            idx[u] = c.start + (uint64_t)(u * kThreads + threadIdx.x) * 4;
            if (idx[u] + 4 <= end) {
                P[u] = ld_nt(t.p + idx[u]);
                G[u] = ld_nt(t.g + idx[u]);
                M[u] = ld_nt(t.m + idx[u]);
                V[u] = ld_nt(t.v + idx[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (idx[u] + 4 <= end) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float pe = P[u][e], me = M[u][e], ve = V[u][e];
                    adam_elem(pe, G[u][e], me, ve, b1, omb1, b2, omb2, eps, step_size,
                              inv_sqrt_bc2);
                    P[u][e] = pe;
                    M[u][e] = me;
                    V[u][e] = ve;
                }
                st_nt(t.p + idx[u], P[u]);
                st_nt(t.m + idx[u], M[u]);
                st_nt(t.v + idx[u], V[u]);
                if (zero_grad) st_nt(t.g + idx[u], f32x4{0.f, 0.f, 0.f, 0.f});
            } else {
                for (uint64_t i = idx[u]; i < end && i < idx[u] + 4; ++i) {
                    float p = t.p[i], m = t.m[i], v = t.v[i];
                    adam_elem(p, t.g[i], m, v, b1, omb1, b2, omb2, eps, step_size,
                              inv_sqrt_bc2);
                    t.p[i] = p;
                    t.m[i] = m;
                    t.v[i] = v;
                    if (zero_grad) t.g[i] = 0.0f;
                }
            }
        }
    } else {
        for (uint64_t i = c.start + threadIdx.x; i < end; i += kThreads) {
            float p = t.p[i], m = t.m[i], v = t.v[i];
            adam_elem(p, t.g[i], m, v, b1, omb1, b2, omb2, eps, step_size, inv_sqrt_bc2);
            t.p[i] = p;
            t.m[i] = m;
            t.v[i] = v;
            if (zero_grad) t.g[i] = 0.0f;
        }
    }
}


// Workgroup w updates chunks w, w + gridDim.x, ...: one chunk each when the
// grid covers the chunk table (a step's single update), several when a
// smaller grid trickles an update beside other kernels.
__global__ __launch_bounds__(kThreads) void adam_mt_dev_kernel(
    const MTTensor *__restrict__ tensors, const MTChunk *__restrict__ chunks, uint32_t nchunks,
    float b1, float b2, float eps, const AdamDevState *__restrict__ st, int zero_grad, int vec) {
    const float step_size = st->step_size, inv_sqrt_bc2 = st->inv_sqrt_bc2;
    for (uint32_t ci = blockIdx.x; ci < nchunks; ci += gridDim.x)
        adam_dev_chunk(tensors, chunks, ci, b1, b2, eps, step_size, inv_sqrt_bc2, zero_grad, vec);
}
// basic_optim.rs:3-31: scaled = g*lr ; w = w - scaled ; g = 0 (fg_optim.h).
__global__ __launch_bounds__(kThreads) void sgd_mt_kernel(const MTTensor *__restrict__ tensors,
                                                          const MTChunk *__restrict__ chunks,
                                                          float lr, int zero_grad, int vec) {
    sgd_chunk(tensors, chunks, lr, zero_grad, vec, blockIdx.x);
}

}  // namespace


FG_API int fg_mt_create_x(fg_ctx *ctx, int n, const int *dtypes, void *const *d_params,
                          void *const *d_grads, float *const *d_m, float *const *d_v,
                          const uint64_t *sizes, fg_mt **out) {
    FG_REQUIRE(ctx && out && n > 0 && d_params && d_grads && sizes, FG_ERR_INVALID_ARGUMENT,
               "fg_mt_create: NULL argument or empty list");
    FG_REQUIRE((d_m == nullptr) == (d_v == nullptr), FG_ERR_INVALID_ARGUMENT,
               "fg_mt_create: pass both m and v lists or neither");
    FG_HIP(hipSetDevice(ctx->device));
    std::vector<MTTensor> tens(n);
    std::vector<MTChunk> chunks;
    bool aligned = true;
    for (int i = 0; i < n; ++i) {
        FG_REQUIRE(d_params[i] && d_grads[i], FG_ERR_INVALID_ARGUMENT,
                   "fg_mt_create: tensor %d has a NULL param or grad", i);
        const int dt = dtypes ? dtypes[i] : FG_DTYPE_F32;
        FG_REQUIRE(dt >= FG_DTYPE_F32 && dt <= FG_DTYPE_BF16, FG_ERR_INVALID_ARGUMENT,
                   "fg_mt_create: tensor %d has unknown dtype %d", i, dt);
        tens[i].p = static_cast<float *>(d_params[i]);
        tens[i].g = static_cast<float *>(d_grads[i]);
        tens[i].m = d_m ? d_m[i] : nullptr;
        tens[i].v = d_v ? d_v[i] : nullptr;
        tens[i].dtype = (uint32_t)dt;
        tens[i].pad = 0;
        if (d_m) {
            FG_REQUIRE(d_m[i] && d_v[i], FG_ERR_INVALID_ARGUMENT,
                       "fg_mt_create: tensor %d has a NULL optimiser state", i);
        }
        tens[i].n = sizes[i];
        auto al = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
        aligned = aligned && al(tens[i].p) && al(tens[i].g) && (!d_m || (al(tens[i].m) && al(tens[i].v)));
        for (uint64_t s = 0; s < sizes[i]; s += kChunk) chunks.push_back(MTChunk{(uint32_t)i, 0u, s});
    }
    FG_REQUIRE(!chunks.empty(), FG_ERR_INVALID_ARGUMENT, "fg_mt_create: all tensors are empty");
    FG_REQUIRE(chunks.size() < (1ull << 31), FG_ERR_OUT_OF_BOUNDS,
               "fg_mt_create: %zu chunks exceed the grid limit", chunks.size());
    fg_mt *mt = new fg_mt;
    mt->device = ctx->device;
    mt->n = n;
    mt->has_state = d_m != nullptr;
    mt->vec = aligned ? 1 : 0;
    mt->nchunks = (uint32_t)chunks.size();
    hipError_t e = hipMalloc(&mt->d_tensors, sizeof(MTTensor) * n);
    if (e == hipSuccess) e = hipMalloc(&mt->d_chunks, sizeof(MTChunk) * chunks.size());
    if (e == hipSuccess)
        e = hipMemcpy(mt->d_tensors, tens.data(), sizeof(MTTensor) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(mt->d_chunks, chunks.data(), sizeof(MTChunk) * chunks.size(),
                      hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(mt->d_tensors);
        (void)hipFree(mt->d_chunks);
        delete mt;
        return fg::hip_fail(e, "fg_mt_create", __FILE__, __LINE__);
    }
    *out = mt;
    return FG_OK;
}

FG_API int fg_mt_create(fg_ctx *ctx, int n, float *const *d_params, float *const *d_grads,
                        float *const *d_m, float *const *d_v, const uint64_t *sizes,
                        fg_mt **out) {
    return fg_mt_create_x(ctx, n, nullptr, reinterpret_cast<void *const *>(d_params),
                          reinterpret_cast<void *const *>(d_grads), d_m, d_v, sizes, out);
}

FG_API int fg_mt_destroy(fg_mt *mt) {
    if (!mt) return FG_OK;
    // hipFree waits for outstanding work on the device; the owning context
    // may already be gone, so it is not touched here.
    (void)hipSetDevice(mt->device);
    (void)hipFree(mt->d_tensors);
    (void)hipFree(mt->d_chunks);
    delete mt;
    return FG_OK;
}

FG_API int fg_sgd_step(fg_ctx *ctx, fg_mt *mt, float lr, int zero_grad) {
    FG_REQUIRE(ctx && mt, FG_ERR_INVALID_ARGUMENT, "fg_sgd_step: NULL argument");
    FG_HIP(hipSetDevice(ctx->device));
    sgd_mt_kernel<<<mt->nchunks, kThreads, 0, ctx->stream>>>(mt->d_tensors, mt->d_chunks, lr,
                                                            zero_grad, mt->vec);
    FG_LAUNCH_CHECK("sgd_mt_kernel");
    return FG_OK;
}

FG_API int fg_adam_step_scalars(fg_ctx *ctx, fg_mt *mt, float b1, float b2, float eps,
                                float step_size, float inv_sqrt_bc2, int zero_grad) {
    FG_REQUIRE(ctx && mt, FG_ERR_INVALID_ARGUMENT, "fg_adam_step: NULL argument");
    FG_REQUIRE(mt->has_state, FG_ERR_INVALID_ARGUMENT,
               "fg_adam_step: tensor list was created without m/v state");
    FG_HIP(hipSetDevice(ctx->device));
    adam_mt_kernel<<<mt->nchunks, kThreads, 0, ctx->stream>>>(
        mt->d_tensors, mt->d_chunks, b1, b2, eps, step_size, inv_sqrt_bc2, zero_grad, mt->vec);
    FG_LAUNCH_CHECK("adam_mt_kernel");
    return FG_OK;
}

namespace fg {

uint64_t adam_dev_state_bytes() { return sizeof(AdamDevState); }

// Advance the device step counter at d_state (zero-initialised
// AdamDevState) and derive the step's bias-correction scalars.
int adam_dev_advance_on(hipStream_t stream, float lr, float b1, float b2, void *d_state) {
    FG_REQUIRE(d_state, FG_ERR_INVALID_ARGUMENT, "adam_dev_advance: NULL state");
    AdamDevState *st = reinterpret_cast<AdamDevState *>(d_state);
    adam_advance_kernel<<<1, 64, 0, stream>>>(st, (double)lr, (double)b1, (double)b2);
    FG_LAUNCH_CHECK("adam_advance_kernel");
    return FG_OK;
}

int adam_dev_advance(fg_ctx *ctx, float lr, float b1, float b2, void *d_state) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "adam_dev_advance: NULL context");
    return adam_dev_advance_on(ctx->stream, lr, b1, b2, d_state);
}

// One Adam update of mt's tensors on `stream` with the scalars at d_state
// (advanced by adam_dev_advance before this runs).
int mt_adam_dev_update(fg_mt *mt, hipStream_t stream, float b1, float b2, float eps,
                       const void *d_state, int zero_grad, uint32_t max_blocks) {
    FG_REQUIRE(mt && d_state, FG_ERR_INVALID_ARGUMENT, "mt_adam_dev_update: NULL argument");
    FG_REQUIRE(mt->has_state, FG_ERR_INVALID_ARGUMENT,
               "mt_adam_dev_update: tensor list was created without m/v state");
    const uint32_t blocks = max_blocks && max_blocks < mt->nchunks ? max_blocks : mt->nchunks;
    adam_mt_dev_kernel<<<blocks, kThreads, 0, stream>>>(
        mt->d_tensors, mt->d_chunks, mt->nchunks, b1, b2, eps,
        reinterpret_cast<const AdamDevState *>(d_state), zero_grad, mt->vec);
    FG_LAUNCH_CHECK("adam_mt_dev_kernel");
    return FG_OK;
}

// Advance the device step counter and apply one Adam update.
int mt_adam_dev(fg_ctx *ctx, fg_mt *mt, float lr, float b1, float b2, float eps, void *d_state,
                int zero_grad) {
    FG_REQUIRE(ctx && mt && d_state, FG_ERR_INVALID_ARGUMENT, "mt_adam_dev: NULL argument");
    if (int rc = adam_dev_advance(ctx, lr, b1, b2, d_state)) return rc;
    return mt_adam_dev_update(mt, ctx->stream, b1, b2, eps, d_state, zero_grad, 0);
}

}  // namespace fg

FG_API int fg_adam_step(fg_ctx *ctx, fg_mt *mt, float lr, float b1, float b2, float eps,
                        int step, int zero_grad) {
    FG_REQUIRE(step >= 1, FG_ERR_INVALID_ARGUMENT, "fg_adam_step: step must be >= 1 (got %d)",
               step);
    const double bc1 = 1.0 - std::pow((double)b1, (double)step);
    const double bc2 = 1.0 - std::pow((double)b2, (double)step);
    const float step_size = (float)((double)lr / bc1);
    const float inv_sqrt_bc2 = (float)(1.0 / std::sqrt(bc2));
    return fg_adam_step_scalars(ctx, mt, b1, b2, eps, step_size, inv_sqrt_bc2, zero_grad);
}
