// fg_bias_grad.h -- column sums of dZ[M][N] (the bias add's backward,
// dbias = sum over rows of dZ; the reference's add has no broadcast and so
// no such reduction, crates/ferrograd-nn/src/op/binary.rs:53-63).
//
// Two passes, deterministic:
//  * bias_grad_partial -- grid (column strips of 256 columns, row splits);
//    each thread sums 4 columns (float4) over its rows of the split; the
//    per-split sums go to a partial buffer [splits][N];
//  * bias_grad_final -- one thread per column adds the splits in order and
//    rounds once to the element type of dbias.
// The split count depends only on (CU count, M, N), so the partial buffer
// size is known before the launch (split_of).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "fg_act.h"
#include "fg_half.h"

namespace fg {
namespace colsum {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kCols = 256;                           // columns per strip (64 lanes x float4)
constexpr int kRowGroups = kThreads / (kCols / 4);  // 4 row groups per strip

struct Split {
    int strips = 0, splits = 0, rows_per_split = 0;
    // Size of the partial buffer: one row of N sums per split.
    uint64_t partial_floats(int N) const { return (uint64_t)splits * (uint64_t)N; }
};

// Enough row splits for ~4 workgroups per CU, each covering >= 16 rows.
inline Split split_of(int cus, int M, int N) {
    Split s;
    s.strips = (N + kCols - 1) / kCols;
    if (M <= 0 || N <= 0) return s;
    int splits = std::max(1, std::min((4 * cus + s.strips - 1) / s.strips, (M + 15) / 16));
    s.rows_per_split = (M + splits - 1) / splits;
    s.splits = (M + s.rows_per_split - 1) / s.rows_per_split;
    return s;
}

// DT: element type of dZ (fg_half.h codes); 16-bit rows are read 4
// elements (8 bytes) at a time when aligned.  PACT != kActNone (fp32 only):
// the rows summed are dZ * act'(Pz) (Pz[M][N], row stride ldp, the same
// alignment as dZ), i.e. the bias gradient below an activation whose
// derivative was not applied yet; with `out` (fp32, row stride ldo, the same
// alignment) the scaled rows are also written there, so one pass
// materialises dZ = dC * act'(Pz) and sums its columns.
template <int DT, int PACT = kActNone>
__global__ __launch_bounds__(kThreads) void bias_grad_partial(const void *__restrict__ dZ, int M,
                                                              int N, int ld, int rows_per_split,
                                                              float *__restrict__ partial,
                                                              int vec,
                                                              const float *__restrict__ Pz = nullptr,
                                                              int ldp = 0,
                                                              float *__restrict__ out = nullptr,
                                                              int ldo = 0) {
    static_assert(PACT == kActNone || DT == fg::kF32, "prologue on fp32 rows only");
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __shared__ f32x4 sh[kThreads];
    const int strip = blockIdx.x, split = blockIdx.y;
    const int cq = threadIdx.x % (kCols / 4);
    const int rg = threadIdx.x / (kCols / 4);
    const int col = strip * kCols + cq * 4;
    const int r0 = split * rows_per_split;
    const int r1 = min(M, r0 + rows_per_split);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if (col < N) {
        for (int r = r0 + rg; r < r1; r += kRowGroups) {
            const uint64_t row = (uint64_t)r * ld;
            if (vec && col + 4 <= N) {
                if constexpr (DT == fg::kF32) {
                    f32x4 v = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(dZ) +
                                                               row + col);
                    if constexpr (PACT != kActNone) {
                        const f32x4 z =
                            *reinterpret_cast<const f32x4 *>(Pz + (uint64_t)r * ldp + col);
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] *= act_grad(PACT, z[e]);
                        if (out) *reinterpret_cast<f32x4 *>(out + (uint64_t)r * ldo + col) = v;
                    }
                    s += v;
                } else {
                    const u32x2 w = *reinterpret_cast<const u32x2 *>(
                        static_cast<const uint16_t *>(dZ) + row + col);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        s[e] += fg::h16_to_f(DT, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (col + e >= N) continue;
                    float v = fg::load_as_f(dZ, DT, row + col + e);
                    if constexpr (PACT != kActNone) {
                        v *= act_grad(PACT, Pz[(uint64_t)r * ldp + col + e]);
                        if (out) out[(uint64_t)r * ldo + col + e] = v;
                    }
                    s[e] += v;
                }
            }
        }
    }
    sh[threadIdx.x] = s;
    __syncthreads();
    if (rg == 0 && col < N) {
        f32x4 t = sh[cq];
#pragma unroll
        for (int g = 1; g < kRowGroups; ++g) t += sh[g * (kCols / 4) + cq];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (col + e < N) partial[(size_t)split * N + col + e] = t[e];
    }
}

// Adds the splits of each column in order; the sum is rounded to the
// element type dt once (with accumulate: round(dbias + sum)).  The partials
// are loaded kBatch at a time before they are added (in the same order), so
// a thread waits for one memory round trip per kBatch splits rather than
// per split.
template <int kBatch = 16>
__global__ __launch_bounds__(kThreads) void bias_grad_final(const float *__restrict__ partial,
                                                            int splits, int N,
                                                            void *__restrict__ dbias,
                                                            int accumulate, int dt) {
    const int col = blockIdx.x * kThreads + threadIdx.x;
    if (col >= N) return;
    float s = 0.0f;
    int k = 0;
    for (; k + kBatch <= splits; k += kBatch) {
        float v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) v[u] = partial[(size_t)(k + u) * N + col];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) s += v[u];
    }
    for (; k < splits; ++k) s += partial[(size_t)k * N + col];
    fg::store_from_f(dbias, dt, col, accumulate ? fg::load_as_f(dbias, dt, col) + s : s);
}

// Enqueues both passes; `partial` holds at least sp.splits * N floats.
// dtype is an FG_DTYPE_* code (the fg_half.h codes coincide).  pact / Pz /
// ldp: the optional prologue of bias_grad_partial (fp32 dZ only; the caller
// checks), and `out` / ldo its optional output of the scaled rows.  dbias
// NULL: the first pass only (out written, no sums kept).
inline hipError_t launch(hipStream_t st, const Split &sp, int dtype, int M, int N,
                         const void *dZ, int ld, void *dbias, int accumulate, float *partial,
                         int pact = kActNone, const float *Pz = nullptr, int ldp = 0,
                         float *out = nullptr, int ldo = 0) {
    const unsigned align = dtype == fg::kF32 ? 16u : 8u;
    int vec = ((((uintptr_t)dZ) & (align - 1)) == 0) && (ld % 4 == 0);
    if (pact != kActNone) vec = vec && (((uintptr_t)Pz) & 15u) == 0 && ldp % 4 == 0;
    if (out) vec = vec && (((uintptr_t)out) & 15u) == 0 && ldo % 4 == 0;
    int splits = sp.splits;
    if (M > 0) {
        const dim3 grid(sp.strips, splits);
        if (pact == kActRelu)
            bias_grad_partial<fg::kF32, kActRelu><<<grid, kThreads, 0, st>>>(
                dZ, M, N, ld, sp.rows_per_split, partial, vec, Pz, ldp, out, ldo);
        else if (pact == kActGelu)
            bias_grad_partial<fg::kF32, kActGelu><<<grid, kThreads, 0, st>>>(
                dZ, M, N, ld, sp.rows_per_split, partial, vec, Pz, ldp, out, ldo);
        else if (dtype == fg::kF32)
            bias_grad_partial<fg::kF32>
                <<<grid, kThreads, 0, st>>>(dZ, M, N, ld, sp.rows_per_split, partial, vec);
        else if (dtype == fg::kF16)
            bias_grad_partial<fg::kF16>
                <<<grid, kThreads, 0, st>>>(dZ, M, N, ld, sp.rows_per_split, partial, vec);
        else
            bias_grad_partial<fg::kBF16>
                <<<grid, kThreads, 0, st>>>(dZ, M, N, ld, sp.rows_per_split, partial, vec);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    } else {
        splits = 0;
    }
    if (!dbias) return hipSuccess;
    bias_grad_final<><<<(N + kThreads - 1) / kThreads, kThreads, 0, st>>>(partial, splits, N,
                                                                         dbias, accumulate, dtype);
    return hipGetLastError();
}

}  // namespace colsum
}  // namespace fg
