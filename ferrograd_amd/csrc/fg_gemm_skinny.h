// fg_gemm_skinny.h -- GEMMs with few output columns and a short K (N <= 16,
// K <= 256), in every layout: the second layer and the head gradients of a
// small MLP (c1: 64x10x256 forward, dW = X^T.dZ of 256x10x64 with its bias
// gradient).  The tiled kernels walk such shapes as a chain of K tiles, one
// memory round trip each, on a handful of workgroups.  Here a workgroup owns
// 16 output rows and every column: it issues all the loads of its A row panel
// and of the whole B panel at once (one round trip), stages them in LDS, and
// sums from there with no K loop of loads, 16 k-groups of at most 16 k in
// parallel.  Deterministic: each output is the 16 group sums (ascending k)
// added in group order.
#pragma once

#include "fg_gemm_kernel.h"
#include "fg_internal.h"
#include "fg_softmax_row.h"

namespace fg {
namespace gemm {

constexpr int kSkRows = 16;              // output rows per workgroup
constexpr int kSkThreads = 256;
constexpr int kSkGroups = kSkThreads / kSkRows;              // K groups: 16
constexpr int kSkAPerThread = kSkRows * kSkinnyK / kSkThreads;  // 16
constexpr int kSkBPerThread = kSkinnyK * kSkinnyN / kSkThreads;  // 16
constexpr int kSkAStride = kSkRows + 1;    // As[k][row], padded
static_assert(kSkinnyN == 16 && kSkinnyK == kSkThreads && kSkGroups == 16,
              "thread layouts below assume these");
inline int skinny_workgroups(int M) { return (M + kSkRows - 1) / kSkRows; }

template <bool AK, bool BNC>
__device__ __forceinline__ void gemm_f32_skinny_body(GemmArgs p, int bx) {
    __shared__ float As[kSkinnyK * kSkAStride];
    __shared__ __attribute__((aligned(16))) float Bs[kSkinnyK * kSkinnyN];
    __shared__ float red[kSkGroups * kSkinnyN * kSkRows];
    const int t = threadIdx.x;
    const int m0 = bx * kSkRows;

    // All loads first (registers), then the LDS stores: one round trip.
    float ra[kSkAPerThread], rb[kSkBPerThread];
    if constexpr (AK) {
        // A[m][k]: thread t holds column k = t of the 16 rows (coalesced in k).
#pragma unroll
        for (int i = 0; i < kSkAPerThread; ++i)
            ra[i] = (t < p.K && m0 + i < p.M) ? p.A[(size_t)(m0 + i) * p.lda + t] : 0.0f;
    } else {
        // A[k][m]: thread t holds row t % 16 at k = t / 16 + 16i (coalesced in m).
        const int r = t % kSkRows, k0 = t / kSkRows;
#pragma unroll
        for (int i = 0; i < kSkAPerThread; ++i) {
            const int k = k0 + kSkGroups * i;
            ra[i] = (k < p.K && m0 + r < p.M) ? p.A[(size_t)k * p.lda + m0 + r] : 0.0f;
        }
    }
    if constexpr (BNC) {
        // B[k][n]: thread t holds column n = t % 16 at k = t / 16 + 16i.
        const int n = t % kSkinnyN, k0 = t / kSkinnyN;
#pragma unroll
        for (int i = 0; i < kSkBPerThread; ++i) {
            const int k = k0 + kSkinnyN * i;
            rb[i] = (k < p.K && n < p.N) ? p.B[(size_t)k * p.ldb + n] : 0.0f;
        }
    } else {
        // B[n][k]: thread t holds k = t of the 16 columns (coalesced in k).
#pragma unroll
        for (int n = 0; n < kSkBPerThread; ++n)
            rb[n] = (t < p.K && n < p.N) ? p.B[(size_t)n * p.ldb + t] : 0.0f;
    }
    if constexpr (AK) {
#pragma unroll
        for (int i = 0; i < kSkAPerThread; ++i) As[t * kSkAStride + i] = ra[i];
    } else {
        const int r = t % kSkRows, k0 = t / kSkRows;
#pragma unroll
        for (int i = 0; i < kSkAPerThread; ++i) As[(k0 + kSkGroups * i) * kSkAStride + r] = ra[i];
    }
    if constexpr (BNC) {
        const int n = t % kSkinnyN, k0 = t / kSkinnyN;
#pragma unroll
        for (int i = 0; i < kSkBPerThread; ++i) Bs[(k0 + kSkinnyN * i) * kSkinnyN + n] = rb[i];
    } else {
#pragma unroll
        for (int n = 0; n < kSkBPerThread; ++n) Bs[t * kSkinnyN + n] = rb[n];
    }
    __syncthreads();

    // Thread (r, g): row r over the g-th K group (at most 16 k), all 16
    // columns.
    {
        const int r = t % kSkRows, g = t / kSkRows;
        const int kg = (p.K + kSkGroups - 1) / kSkGroups;
        const int kb = g * kg, ke = min(p.K, kb + kg);
        float acc[kSkinnyN];
#pragma unroll
        for (int n = 0; n < kSkinnyN; ++n) acc[n] = 0.0f;
        for (int k = kb; k < ke; ++k) {
            const float a = As[k * kSkAStride + r];
            const f32x4 *b = reinterpret_cast<const f32x4 *>(Bs + k * kSkinnyN);
#pragma unroll
            for (int j = 0; j < kSkinnyN / 4; ++j) {
                const f32x4 bj = b[j];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[4 * j + e] += a * bj[e];
            }
        }
#pragma unroll
        for (int n = 0; n < kSkinnyN; ++n) red[(g * kSkinnyN + n) * kSkRows + r] = acc[n];
    }
    // Bias gradient (TN with colsum): workgroup 0 sums each column of the B
    // panel, 16 k-groups in ascending k, then the groups in order.
    const bool do_cs = p.colsum && bx == 0;
    float csum = 0.0f;
    if (do_cs) {
        const int n = t % kSkinnyN, g = t / kSkinnyN;
        for (int k = g; k < p.K; k += kSkinnyN) csum += Bs[k * kSkinnyN + n];
    }
    __syncthreads();

    // Epilogue: thread (r, n) finishes output (m0 + r, n): the 16 K-group
    // sums in group order.
    {
        const int r = t % kSkRows, col = t / kSkRows;
        const int row = m0 + r;
        if (row < p.M && col < p.N) {
            float v = red[col * kSkRows + r];
#pragma unroll
            for (int g = 1; g < kSkGroups; ++g) v += red[(g * kSkinnyN + col) * kSkRows + r];
            const float b = (p.mode == 0 && p.bias) ? p.bias[col] : 0.0f;
            float z;
            float o = epi_value(p, v, b, row, col, &z);
            if (p.mode == 0 && p.Z) p.Z[(size_t)row * p.ldz + col] = z;
            float *c = p.C + (size_t)row * p.ldc + col;
            if (p.accumulate) o += *c;
            *c = o;
        }
    }
    if (do_cs) {
        // The 16 k-group sums of each column, through the (now free) B panel.
        __syncthreads();
        Bs[t] = csum;  // [group][n]
        __syncthreads();
        if (t < p.N) {
            float s = Bs[t];
            for (int g = 1; g < kSkThreads / kSkinnyN; ++g) s += Bs[g * kSkinnyN + t];
            p.colsum[t] = p.colsum_accumulate ? p.colsum[t] + s : s;
        }
    }
}

// NN with a summing prologue: A is the output of a split-K GEMM `pre` whose
// slices have not been summed.  A workgroup owns kSpRows output rows, a
// quarter of the plain kernel's, so the slices' bytes spread over four
// times as many CUs (one CU pulls them at a few tens of GB/s).  It sums its
// rows' slices in slice order, applies pre's epilogue (bias, activation, Z)
// and writes pre's outputs -- per element the operations of splitk_reduce,
// so the same bits -- and takes its A panel from those values.  The product
// is then exactly the plain kernel's (16 k-groups of the same extent, each
// in ascending k, the group sums added in group order), so the same bits as
// gemm_f32_skinny_body.  Host conditions (fg::gemm_fwd_chain_f32): at most
// kSkPreMaxSlices slices, pre's N (this GEMM's K) a multiple of 4, pre's
// rows 16-byte aligned (pre.vec_out).
//
// With CE the outputs are a head's logits (N <= 16 columns, forward
// epilogue, no accumulation) and the workgroup also finishes the softmax +
// cross-entropy of its rows: wave 0 holds them as four 16-lane row groups
// and runs the one-workgroup loss kernel's row code (fg::smrow::ce_row16),
// writing dlogits, the row losses and the probabilities exactly as that
// kernel would from the stored logits.
constexpr int kSpRows = 4;
static_assert(kSpRows * kSkinnyK == 4 * kSkThreads, "one float4 of A per thread");
inline int skinny_pre_workgroups(int M) { return (M + kSpRows - 1) / kSpRows; }

template <bool CE = false>
__device__ __forceinline__ void gemm_f32_skinny_pre_body(const GemmArgs &p, const GemmArgs &pre,
                                                         int bx, const CeOut &ce) {
    static_assert(kSkinnyN == smrow::kCols && kSpRows * smrow::kCols == 64,
                  "one wave holds the workgroup's rows as 16-lane groups");
    __shared__ float As[kSkinnyK * kSpRows];  // As[k][r]
    __shared__ __attribute__((aligned(16))) float Bs[kSkinnyK * kSkinnyN];
    __shared__ float red[kSkGroups * kSkinnyN * kSpRows];
    const int t = threadIdx.x;
    const int m0 = bx * kSpRows;

    // Every load first: thread t holds columns c4..c4+3 of local row r, all
    // slices, and its part of the B panel (B[k][n]).
    const int c4 = 4 * (t % (kSkinnyK / 4)), r = t / (kSkinnyK / 4);
    const int row = m0 + r;
    const int S = (pre.K + pre.ksplit - 1) / pre.ksplit;
    const bool ok = row < pre.M && c4 < pre.N;
    const float *src = pre.partial + (size_t)row * pre.N + c4;
    const size_t mn = (size_t)pre.M * pre.N;
    f32x4 sl[kSkPreMaxSlices];
#pragma unroll
    for (int s = 0; s < kSkPreMaxSlices; ++s)
        sl[s] = (ok && s < S) ? *reinterpret_cast<const f32x4 *>(src + s * mn)
                              : f32x4{0.f, 0.f, 0.f, 0.f};
    float rb[kSkBPerThread];
    const int bn = t % kSkinnyN, bk0 = t / kSkinnyN;
#pragma unroll
    for (int i = 0; i < kSkBPerThread; ++i) {
        const int k = bk0 + kSkinnyN * i;
        rb[i] = (k < p.K && bn < p.N) ? p.B[(size_t)k * p.ldb + bn] : 0.0f;
    }
    const f32x4 bv = (pre.bias && c4 < pre.N) ? *reinterpret_cast<const f32x4 *>(pre.bias + c4)
                                              : f32x4{0.f, 0.f, 0.f, 0.f};

    // pre's outputs: the slices in slice order, then pre's epilogue.  With
    // CE and a data gradient, pre's Z values (v + bias, as epi_x4 stores
    // them) are kept for the act' of that gradient.
    __shared__ float zsh[CE ? kSpRows * kSkinnyK : 1];
    f32x4 h = {0.f, 0.f, 0.f, 0.f};
    if (ok) {
        f32x4 v = sl[0];
#pragma unroll
        for (int s = 1; s < kSkPreMaxSlices; ++s)
            if (s < S) v += sl[s];
        if constexpr (CE) {
            const f32x4 z = v + bv;
#pragma unroll
            for (int e = 0; e < 4; ++e) zsh[r * kSkinnyK + c4 + e] = z[e];
        }
        h = epi_x4(pre, v, bv, row, c4);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) As[(c4 + e) * kSpRows + r] = h[e];
#pragma unroll
    for (int i = 0; i < kSkBPerThread; ++i) Bs[(bk0 + kSkinnyN * i) * kSkinnyN + bn] = rb[i];
    __syncthreads();

    // The plain kernel's sums: thread (r, g) = (t % kSpRows, t / kSpRows)
    // takes row r over the g-th K group, all 16 columns.
    if (t < kSpRows * kSkGroups) {
        const int rr = t % kSpRows, g = t / kSpRows;
        const int kg = (p.K + kSkGroups - 1) / kSkGroups;
        const int kb = g * kg, ke = min(p.K, kb + kg);
        float acc[kSkinnyN];
#pragma unroll
        for (int n = 0; n < kSkinnyN; ++n) acc[n] = 0.0f;
        for (int k = kb; k < ke; ++k) {
            const float a = As[k * kSpRows + rr];
            const f32x4 *b = reinterpret_cast<const f32x4 *>(Bs + k * kSkinnyN);
#pragma unroll
            for (int j = 0; j < kSkinnyN / 4; ++j) {
                const f32x4 bj = b[j];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[4 * j + e] += a * bj[e];
            }
        }
#pragma unroll
        for (int n = 0; n < kSkinnyN; ++n) red[(g * kSkinnyN + n) * kSpRows + rr] = acc[n];
    }
    __syncthreads();

    // Epilogue: thread (r, n) finishes output (m0 + r, n).
    __shared__ float logits[CE ? kSpRows * kSkinnyN : 1];
    if (t < kSpRows * kSkinnyN) {
        const int rr = t % kSpRows, col = t / kSpRows;
        const int orow = m0 + rr;
        if (orow < p.M && col < p.N) {
            float v = red[col * kSpRows + rr];
#pragma unroll
            for (int g = 1; g < kSkGroups; ++g) v += red[(g * kSkinnyN + col) * kSpRows + rr];
            const float b = (p.mode == 0 && p.bias) ? p.bias[col] : 0.0f;
            float z;
            float o = epi_value(p, v, b, orow, col, &z);
            if (p.mode == 0 && p.Z) p.Z[(size_t)orow * p.ldz + col] = z;
            float *c = p.C + (size_t)orow * p.ldc + col;
            if (p.accumulate) o += *c;
            *c = o;
            if constexpr (CE) logits[rr * kSkinnyN + col] = o;
        }
    }
    if constexpr (CE) {
        __shared__ float dl[kSpRows * smrow::kCols];
        __syncthreads();
        if (t < 64) {  // wave 0: lane 16 r + c holds column c of local row r
            const int r = t / smrow::kCols, c = t % smrow::kCols, row = m0 + r;
            const bool valid = row < p.M;
            const float v = (valid && c < p.N) ? logits[r * kSkinnyN + c] : -INFINITY;
            const uint32_t lab = valid ? ce.labels[row] : 0u;
            float d;
            (void)smrow::ce_row16<kF32>(v, lab, c, p.N, row, valid, true, ce.scale, ce.row_loss,
                                        ce.dlogits, ce.ldd, nullptr, ce.probs, ce.ldp, true, &d);
            dl[t] = d;
        }
        if (ce.dz) {
            // dz rows m0.. = (dlogits . B^T) * act'(Z): an NT product of
            // K = p.N (classes) and N = p.K (this GEMM's K).  Wave w takes
            // 32-column blocks 2w, 2w + 1 with the 64x64 kernels' MFMA
            // sequence for one 16-deep K tile (lane half h feeds k = 8h + 4g
            // + s to the s-th MFMA of group g); A rows past the workgroup's
            // four are zero, which leaves its rows' sums unchanged.
            __syncthreads();
            const int lane = t & 63, wave = t >> 6, l32 = lane & 31, hh = lane >> 5;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int n0 = 32 * (2 * wave + jj);
                if (n0 >= p.K) break;  // uniform
                const int n = n0 + l32;
                f32x16 acc;
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
                for (int g = 0; g < 2; ++g) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const int k = 8 * hh + 4 * g + s;
                        const float av = l32 < kSpRows ? dl[l32 * smrow::kCols + k] : 0.0f;
                        const float bw = n < p.K ? Bs[n * kSkinnyN + k] : 0.0f;
                        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bw, acc, 0, 0, 0);
                    }
                }
                // Register r (< 4) of lane half 0 holds row r, column n.
                if (hh == 0 && n < p.K) {
#pragma unroll
                    for (int r = 0; r < kSpRows; ++r) {
                        const int row = m0 + r;
                        if (row >= p.M) continue;
                        float o = acc[r];
                        if (ce.dz_act != kActNone) o *= act_grad(ce.dz_act, zsh[r * kSkinnyK + n]);
                        ce.dz[(size_t)row * ce.lddz + n] = o;
                    }
                }
            }
        }
    }
}

}  // namespace gemm
}  // namespace fg
