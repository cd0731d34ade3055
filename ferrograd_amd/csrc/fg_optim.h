// fg_optim.h -- the multi-tensor optimiser lists of k_optim.hip and the SGD
// update of one chunk, shared with the launch that runs SGD beside a held
// split-K summing pass (k_gemm.hip, fg::sgd_step_with_pending).
#pragma once

#include <hip/hip_runtime.h>

#include "fg_half.h"
#include "fg_internal.h"

namespace fg {
namespace optim {

constexpr int kThreads = 256;
// float4 per thread per stream, and so the chunk of a workgroup: one float4
// (1024-element chunks) streams Adam at 6.15 TB/s and SGD at 6.25 TB/s on
// MI355X, against 5.84 / 5.85 with four (4096) and 5.65 / 5.85 with two.  A
// knob for measurement builds.
#ifndef FG_OPTIM_UNROLL
#define FG_OPTIM_UNROLL 1
#endif
constexpr int kUnroll = FG_OPTIM_UNROLL;
constexpr int kChunk = kThreads * 4 * kUnroll;  // elements per workgroup

// p and g are of element type dtype (fg_half.h codes; 16-bit tensors are
// addressed as 16-bit words through the same pointers); m and v are fp32.
struct MTTensor {
    float *p;
    float *g;
    float *m;
    float *v;
    uint64_t n;
    uint32_t dtype;
    uint32_t pad;
};

struct MTChunk {
    uint32_t tensor;
    uint32_t pad;
    uint64_t start;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ inline f32x4 ld_nt(const float *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
}
__device__ inline void st_nt(float *p, f32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(p));
}

// basic_optim.rs:3-31: scaled = g*lr ; w = w - scaled ; g = 0, over chunk
// `chunk` of the list.  Rounded where written (no contraction of g*lr into
// the subtraction), whatever unit includes it: bit-exact with the CPU
// restatement.
__device__ __forceinline__ void sgd_chunk(const MTTensor *__restrict__ tensors,
                                          const MTChunk *__restrict__ chunks, float lr,
                                          int zero_grad, int vec, uint32_t chunk) {
#pragma clang fp contract(off)
    const MTChunk c = chunks[chunk];
    const MTTensor t = tensors[c.tensor];
    const uint64_t end = (c.start + kChunk < t.n) ? c.start + kChunk : t.n;
    if (t.dtype != fg::kF32) {  // 16-bit: w = round(w - g*lr)
        uint16_t *w16 = reinterpret_cast<uint16_t *>(t.p);
        uint16_t *g16 = reinterpret_cast<uint16_t *>(t.g);
        for (uint64_t i = c.start + threadIdx.x; i < end; i += kThreads) {
            const float w = fg::h16_to_f(t.dtype, w16[i]), g = fg::h16_to_f(t.dtype, g16[i]);
            w16[i] = fg::f_to_h16(t.dtype, w - g * lr);
            if (zero_grad) g16[i] = 0;
        }
        return;
    }
    if (vec) {
        f32x4 W[kUnroll], G[kUnroll];
        uint64_t idx[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            idx[u] = c.start + (uint64_t)(u * kThreads + threadIdx.x) * 4;
            if (idx[u] + 4 <= end) {
                W[u] = ld_nt(t.p + idx[u]);
                G[u] = ld_nt(t.g + idx[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (idx[u] + 4 <= end) {
#pragma unroll
                for (int e = 0; e < 4; ++e) W[u][e] = W[u][e] - G[u][e] * lr;
                st_nt(t.p + idx[u], W[u]);
                if (zero_grad) st_nt(t.g + idx[u], f32x4{0.f, 0.f, 0.f, 0.f});
            } else {
                for (uint64_t i = idx[u]; i < end && i < idx[u] + 4; ++i) {
                    t.p[i] = t.p[i] - t.g[i] * lr;
                    if (zero_grad) t.g[i] = 0.0f;
                }
            }
        }
    } else {
        for (uint64_t i = c.start + threadIdx.x; i < end; i += kThreads) {
            t.p[i] = t.p[i] - t.g[i] * lr;
            if (zero_grad) t.g[i] = 0.0f;
        }
    }
}

}  // namespace optim
}  // namespace fg

struct fg_mt {
    int device = 0;
    int n = 0;
    bool has_state = false;
    int vec = 0;
    uint32_t nchunks = 0;
    fg::optim::MTTensor *d_tensors = nullptr;
    fg::optim::MTChunk *d_chunks = nullptr;
};
