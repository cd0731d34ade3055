// fg_gemm16_kernel.h -- 16-bit (bf16 / fp16) GEMM on CDNA4 matrix cores
// (v_mfma_f32_32x32x16_bf16 / _f16) with fp32 accumulation and the same
// fused epilogues as the fp32 kernel.  Included by k_gemm16_{bf16,f16}.hip.
//
// The reference evaluates a 16-bit matmul with its accumulator declared in
// the node's type (crates/ferrograd-nn/src/op/matmul/mod.rs:150-161,
// generic.rs:251-314), i.e. a 16-bit running sum over K.  Here products are
// summed in fp32 and the result is rounded once to the storage type; then,
// as the reference's node values are, the bias-add node and the activation
// node are each rounded to the storage type.
//
// Design of gemm16_mfma, the kernel for any shape (gfx950; the pipelined
// kernel for whole tiles, gemm16_pipe, is described at its definition):
//  * Each MFMA consumes, per lane, 8 consecutive k of one row of A and of
//    one column of B (16 bytes each).  Both operands are therefore kept in
//    LDS k-contiguous, [row][k] with a row stride of BK+8 elements (16-byte
//    aligned rows, conflict-free 16-byte reads).  An operand that is
//    row-contiguous in memory (B of NN, both operands of TN) is transposed
//    on its way to LDS: a thread loads a 4(k) x 8(row) block with four
//    16-byte loads and writes eight 8-byte k-runs, built with v_perm_b32.
//  * K advances in BK-deep tiles through double-buffered LDS (one barrier
//    per tile); the global loads of tile t+1 are in flight during the MFMAs
//    of tile t.
//  * Accumulators (TM x TN blocks of 16 fp32 per lane) are staged through
//    LDS one 32-row slice at a time for the epilogue, which reads bias / Z
//    and writes C / Z four elements (8 bytes) per lane.
//  * Workgroup ids are remapped per XCD as in the fp32 kernel.
#pragma once

#include <hip/hip_runtime.h>

#include "fg_act.h"
#include "fg_half.h"
#include "fg_sched.h"

namespace fg {
namespace gemm16 {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct Args {
    const uint16_t *A;
    const uint16_t *B;
    uint16_t *C;
    uint16_t *Z;           // forward: pre-activation output (optional)
    const uint16_t *bias;  // forward: row-broadcast bias (optional)
    const uint16_t *Zs;    // backward: saved pre-activation for act'(.)
    int M, N, K;
    int lda, ldb, ldc, ldz, ldzs;
    int act;
    int mode;  // 0 forward epilogue, 1 backward (act-derivative) epilogue
    int accumulate;
    int tiles_m, tiles_n;
    int vec_out;  // C / Z / Zs rows and bias 8-byte aligned: 4-element epilogue I/O
    // TN on the pipelined path only: colsum[n] (=|+=) sum_k B[k][n] --
    // the bias gradient of the layer whose weight gradient this GEMM
    // computes -- summed in fp32 from the B tiles already in LDS by the
    // workgroups of the first tile row, rounded to the storage type once.
    uint16_t *colsum;
    int colsum_accumulate;
    // K split (pipelined kernel only, never with colsum): workgroup row s
    // (blockIdx.y) multiplies K elements [s * ksplit, (s + 1) * ksplit) and
    // writes its fp32 sums, without epilogue, into the M x N slot s of
    // partial (row length N); sum_slices16 then adds the slots in slot order
    // and applies the epilogue.  ksplit 0: no split.
    float *partial;
    int ksplit;
    // With colsum and a K split: slot s of N fp32 column sums of the slice,
    // added in slot order, rounded and written (or accumulated) by
    // sum_slices16.
    float *colsum_partial;
};

// Element conversion and the MFMA of one storage type.  from_f rounds the
// fp32 value it is given: an empty asm statement keeps the compiler from
// folding the operation that produced it into the conversion (fp16 has
// v_fma_mix*, which computed GELU's z * s as fma(s, z, +0) and so returned
// +0 where the product is -0), so every epilogue rounds the same fp32
// value.
template <bool BF>
struct T16;
__device__ __forceinline__ float opaque(float f) {
    asm volatile("" : "+v"(f));
    return f;
}
template <>
struct T16<true> {
    static __device__ __forceinline__ float to_f(uint16_t h) { return bf16_to_f(h); }
    static __device__ __forceinline__ uint16_t from_f(float f) { return f_to_bf16(opaque(f)); }
    static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};
template <>
struct T16<false> {
    static __device__ __forceinline__ float to_f(uint16_t h) { return f16_to_f(h); }
    static __device__ __forceinline__ uint16_t from_f(float f) { return f_to_f16(opaque(f)); }
    static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
    return (uint32_t)lo | ((uint32_t)hi << 16);
}

// Loads one operand tile (R rows x BK k) into registers and writes it to
// LDS as [row][k] with row stride BK+8.  KC: k-contiguous in memory.
template <int R, int BK, bool KC, bool VEC, int NT>
struct Loader {
    static constexpr int kLd = BK + 8;
    static constexpr int kUnits = KC ? R * BK / 8 : (BK / 4) * (R / 8);
    // Units per thread; when the tile has fewer units than threads, the
    // threads past the last unit load and store nothing.
    static constexpr int kPer = (kUnits + NT - 1) / NT;
    static_assert(kUnits % NT == 0 || kUnits < NT, "tile not divisible by the thread count");
    static __device__ __forceinline__ bool active(int idx) { return kUnits >= NT || idx < kUnits; }
    u32x4 v[KC ? kPer : 4 * kPer];

    __device__ __forceinline__ void load(const uint16_t *__restrict__ base, int ld, int row0,
                                         int rmax, int k0, int K) {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int idx = threadIdx.x + q * NT;
            if (!active(idx)) continue;
            if constexpr (KC) {
                const int row = idx / (BK / 8), kk = (idx % (BK / 8)) * 8;
                const int gr = row0 + row, gk = k0 + kk;
                const uint16_t *p = base + (size_t)gr * ld + gk;
                if (VEC && gr < rmax && gk + 8 <= K) {
                    v[q] = *reinterpret_cast<const u32x4 *>(p);
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) e[t] = (gr < rmax && gk + t < K) ? p[t] : 0;
                    v[q] = u32x4{pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]),
                                 pack2(e[6], e[7])};
                }
            } else {
                const int kq = idx / (R / 8), r8 = idx % (R / 8);
                const int gr = row0 + r8 * 8;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int gk = k0 + kq * 4 + t;
                    const uint16_t *p = base + (size_t)gk * ld + gr;
                    if (VEC && gk < K && gr + 8 <= rmax) {
                        v[q * 4 + t] = *reinterpret_cast<const u32x4 *>(p);
                    } else {
                        uint16_t e[8];
#pragma unroll
                        for (int s = 0; s < 8; ++s) e[s] = (gk < K && gr + s < rmax) ? p[s] : 0;
                        v[q * 4 + t] = u32x4{pack2(e[0], e[1]), pack2(e[2], e[3]),
                                             pack2(e[4], e[5]), pack2(e[6], e[7])};
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void store(uint16_t *lds) const {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int idx = threadIdx.x + q * NT;
            if (!active(idx)) continue;
            if constexpr (KC) {
                const int row = idx / (BK / 8), kk = (idx % (BK / 8)) * 8;
                *reinterpret_cast<u32x4 *>(lds + row * kLd + kk) = v[q];
            } else {
                const int kq = idx / (R / 8), r8 = idx % (R / 8);
                // v[q*4+t] holds k = 4kq+t for rows 8r8..8r8+7 (two rows per
                // dword, the lower row in the low half).  Row e gets the
                // four k as two dwords (k, k+1) and (k+2, k+3).
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int w = e >> 1;
                    const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
                    const uint32_t d0 =
                        __builtin_amdgcn_perm(v[q * 4 + 1][w], v[q * 4 + 0][w], sel);
                    const uint32_t d1 =
                        __builtin_amdgcn_perm(v[q * 4 + 3][w], v[q * 4 + 2][w], sel);
                    *reinterpret_cast<u32x2 *>(lds + (r8 * 8 + e) * kLd + kq * 4) =
                        u32x2{d0, d1};
                }
            }
        }
    }
};

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int nt = tiles_m * tiles_n;
    if ((nt & 7) == 0) bid = (bid & 7) * (nt >> 3) + (bid >> 3);
    constexpr int kGroupM = 4;
    const int per_group = kGroupM * tiles_n;
    const int g = bid / per_group;
    const int first = g * kGroupM;
    const int gsize = min(tiles_m - first, kGroupM);
    const int in = bid - g * per_group;
    tm = first + in % gsize;
    tn = in / gsize;
}

// Epilogue of one element: v is the fp32 sum; node values are rounded to
// the storage type as the reference's matmul, bias-add and activation nodes
// each are.
template <bool BF>
__device__ __forceinline__ float epi16(const Args &p, float v, const uint16_t *bias, int row,
                                       int col, float *zout) {
    using E = T16<BF>;
    v = E::to_f(E::from_f(v));
    if (p.mode == 0) {
        if (bias) v = E::to_f(E::from_f(v + E::to_f(bias[col])));
        *zout = v;
        return p.act == kActNone ? v : E::to_f(E::from_f(act_fwd(p.act, v)));
    }
    if (p.act != kActNone) {
        const float z = E::to_f(p.Zs[(size_t)row * p.ldzs + col]);
        // ReLU' masks (a select: +0 where z <= 0); GELU' scales.
        v = p.act == kActRelu ? (z > 0.0f ? v : 0.0f)
                              : E::to_f(E::from_f(v * act_grad(p.act, z)));
    }
    return v;
}

// Four consecutive outputs of one row (the vector path of the epilogue):
// the same operation sequence as epi16 per element, with the uniform
// choices (mode, activation, bias, accumulate) taken once per four.
template <bool BF>
__device__ __forceinline__ void epi16_x4(const Args &p, f32x4 v, f32x4 bv, int row, int col) {
    using E = T16<BF>;
    auto rnd = [](f32x4 x) {
#pragma unroll
        for (int t = 0; t < 4; ++t) x[t] = E::to_f(E::from_f(x[t]));
        return x;
    };
    auto ld4 = [](const uint16_t *q) {
        const u32x2 w = *reinterpret_cast<const u32x2 *>(q);
        return f32x4{E::to_f((uint16_t)w[0]), E::to_f((uint16_t)(w[0] >> 16)),
                     E::to_f((uint16_t)w[1]), E::to_f((uint16_t)(w[1] >> 16))};
    };
    auto st4 = [](uint16_t *q, f32x4 x) {
        *reinterpret_cast<u32x2 *>(q) = u32x2{pack2(E::from_f(x[0]), E::from_f(x[1])),
                                              pack2(E::from_f(x[2]), E::from_f(x[3]))};
    };
    v = rnd(v);
    if (p.mode == 0) {
        if (p.bias) v = rnd(v + bv);
        if (p.Z) st4(p.Z + (size_t)row * p.ldz + col, v);
        if (p.act != kActNone) {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = act_fwd(p.act, v[t]);
            v = rnd(v);
        }
    } else if (p.act != kActNone) {
        const f32x4 z = ld4(p.Zs + (size_t)row * p.ldzs + col);
        if (p.act == kActRelu) {
            // ReLU' masks (a select: +0 where z <= 0).
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = z[t] > 0.0f ? v[t] : 0.0f;
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = v[t] * act_grad(p.act, z[t]);
            v = rnd(v);
        }
    }
    uint16_t *c = p.C + (size_t)row * p.ldc + col;
    if (p.accumulate) v += ld4(c);
    st4(c, v);
}

// A K slice's raw sums: four (or the last few) fp32 values of one row of
// its slot.  The slot's rows are N floats from a 256-byte aligned base.
__device__ __forceinline__ void store_slice16(const Args &p, f32x4 v, int row, int col) {
    float *q = p.partial + (size_t)row * p.N + col;
    if (p.N % 4 == 0) {
        *reinterpret_cast<f32x4 *>(q) = v;
    } else {
#pragma unroll 1
        for (int t = 0; t < 4 && col + t < p.N; ++t) q[t] = v[t];
    }
}

// Epilogue shared by the 16-bit kernels.  Accumulator register r of lane
// (h, l32) in block (i, j) holds C[r0 + 32i + 8(r/4) + 4h + r%4][c0 + 32j + l32];
// each wave stages one 32 x WTN slice of fp32 sums in LDS (stride WTN+4)
// and writes four outputs (8 bytes) per lane.  A lane keeps the same four
// columns through the slice (its bias is loaded once) and reads the next
// row group from LDS while it processes the current one.  Each CU runs the
// epilogue once per launch, so its code is fetched cold: the uniform
// choices sit outside the per-element arithmetic and the row loop stays
// rolled.  lds must hold NW * 32 * (WTN + 4) floats and be free.
template <bool BF, int TM, int TN, int WTN, int NW>
__device__ __forceinline__ void store_tile16(const Args &p, const f32x16 (&acc)[TM][TN],
                                             float *lds, int r0, int c0, int wave, int lane) {
    using E = T16<BF>;
    constexpr int kStageLd = WTN + 4;
    const int l32 = lane & 31, h = lane >> 5;
    float *stage = lds + wave * (32 * kStageLd);
    constexpr int G4 = WTN / 4;    // groups of 4 columns per slice row
    constexpr int RPP = 64 / G4;   // slice rows per pass of the wave
    constexpr int NP = 32 / RPP;   // passes per slice
    static_assert(64 % G4 == 0 && 32 % RPP == 0, "epilogue lane mapping");
    const int c4 = (lane % G4) * 4, rr0 = lane / G4;
    const int col = c0 + c4;
    const bool vec = p.vec_out && col + 4 <= p.N;
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (p.mode == 0 && p.bias && vec) {
        const u32x2 w = *reinterpret_cast<const u32x2 *>(p.bias + col);
        bv = f32x4{E::to_f((uint16_t)w[0]), E::to_f((uint16_t)(w[0] >> 16)),
                   E::to_f((uint16_t)w[1]), E::to_f((uint16_t)(w[1] >> 16))};
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                stage[((r >> 2) * 8 + h * 4 + (r & 3)) * kStageLd + j * 32 + l32] = acc[i][j][r];
        __syncthreads();
        f32x4 nxt = *reinterpret_cast<const f32x4 *>(stage + rr0 * kStageLd + c4);
#pragma unroll 1
        for (int q = 0; q < NP; ++q) {
            const f32x4 v = nxt;
            if (q + 1 < NP)
                nxt = *reinterpret_cast<const f32x4 *>(stage + (rr0 + (q + 1) * RPP) * kStageLd + c4);
            const int row = r0 + i * 32 + rr0 + q * RPP;
            if (row >= p.M || col >= p.N) continue;
            if (p.ksplit > 0) {
                store_slice16(p, v, row, col);
            } else if (vec) {
                epi16_x4<BF>(p, v, bv, row, col);
            } else {
                uint16_t *crow = p.C + (size_t)row * p.ldc;
                const uint16_t *bias = p.mode == 0 ? p.bias : nullptr;
#pragma unroll 1
                for (int t = 0; t < 4 && col + t < p.N; ++t) {
                    float zt;
                    float ot = epi16<BF>(p, v[t], bias, row, col + t, &zt);
                    if (p.mode == 0 && p.Z) p.Z[(size_t)row * p.ldz + col + t] = E::from_f(zt);
                    if (p.accumulate) ot += E::to_f(crow[col + t]);
                    crow[col + t] = E::from_f(ot);
                }
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------ register epilogue
// The pipelined kernels' epilogue when the workgroup's whole tile is in
// bounds (and rows are 8-byte aligned): no LDS and no workgroup barrier.
// Accumulator registers 4k .. 4k+3 of lane (h, l32) hold rows 8k + 4h + 0..3
// of column l32 of a 32x32 block; within each quad of lanes (l32 = 4a + e)
// a 4x4 transpose by two DPP exchanges leaves lane e with row 8k + 4h + e,
// columns 4a .. 4a+3, which it finishes and stores as 8 bytes (16 for the
// fp32 sums of a K slice).  The kind of epilogue (mode, bias, activation) is
// a template parameter, so the per-element code branches on none of them;
// the operations per element are epi16_x4's, so the bits are those of the
// staged epilogue (store_tile16), which stays for partial tiles.  The
// staged epilogue cost 13 us of a 4096x4096 launch (its LDS round trip,
// barriers and a pass loop branching on every epilogue choice); against it
// (bf16, A/B in one process): c5 hidden forward / dX / dW 75.4 / 72.6 /
// 71.2 -> 73.2 / 70.3 / 67.0 us, their dW + dX pair 140.8 -> 134.3 us,
// 4096^3 NN 116.0 -> 112.9 us, 4096x4096x1024 with bias + GELU + Z 53.4 ->
// 46.7 us.

// epi16_x4 with the mode (0 forward, 1 act-derivative), the bias and the
// activation fixed, without the stores: returns the four C values and (MODE
// 0 with Z) the four Z values, packed; z: the four saved pre-activations
// (MODE 1 with an activation); c_old: C's current four values when
// accumulating.
template <bool BF, int MODE, bool BIAS, int ACT>
__device__ __forceinline__ u32x2 epi16_x4_k(const Args &p, f32x4 v, f32x4 bv, f32x4 z,
                                            f32x4 c_old, u32x2 *zpack) {
    using E = T16<BF>;
    auto rnd = [](f32x4 x) {
#pragma unroll
        for (int t = 0; t < 4; ++t) x[t] = E::to_f(E::from_f(x[t]));
        return x;
    };
    auto pk = [](f32x4 x) {
        return u32x2{pack2(E::from_f(x[0]), E::from_f(x[1])), pack2(E::from_f(x[2]), E::from_f(x[3]))};
    };
    v = rnd(v);
    if constexpr (MODE == 0) {
        if constexpr (BIAS) v = rnd(v + bv);
        *zpack = pk(v);
        if constexpr (ACT != kActNone) {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = act_fwd(ACT, v[t]);
            v = rnd(v);
        }
    } else if constexpr (ACT == kActRelu) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = z[t] > 0.0f ? v[t] : 0.0f;
    } else if constexpr (ACT != kActNone) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = v[t] * act_grad(ACT, z[t]);
        v = rnd(v);
    }
    if (p.accumulate) v += c_old;
    return pk(v);
}

__device__ __forceinline__ f32x4 unpack4(bool bf, u32x2 w) {
    return bf ? f32x4{bf16_to_f((uint16_t)w[0]), bf16_to_f((uint16_t)(w[0] >> 16)),
                      bf16_to_f((uint16_t)w[1]), bf16_to_f((uint16_t)(w[1] >> 16))}
              : f32x4{f16_to_f((uint16_t)w[0]), f16_to_f((uint16_t)(w[0] >> 16)),
                      f16_to_f((uint16_t)w[1]), f16_to_f((uint16_t)(w[1] >> 16))};
}

// The register epilogue over block pairs (j, j+1), whose columns make
// 128-byte rows of C: after the quad transposes, lane (h, a, e) holds row
// 8k + 4h + e of both blocks (8 bytes each); half h sends the other half
// the block it does not store (__shfl_xor by 32), so that lanes of half h
// store block j + h of rows 8k + e and 8k + 4 + e -- every store
// instruction then writes whole 128-byte lines (4 rows).  Storing 64-byte
// halves of lines from different instructions made the bf16 c5 step's Adam
// update that follows the backward 379 -> 414 us.  MODE 2: the raw fp32
// sums of a K slice into its slot, 16 bytes a row per block (whole 128-byte
// lines already).  Blocks (i, pair) are unrolled; the four row groups k of a
// block run as a loop that picks its registers by k, which keeps the code
// (fetched cold, once per CU and launch) short.  MODE 1 with an activation
// loads a block pair's saved pre-activations before its loop.
template <bool BF, int TM, int TN, int MODE, bool BIAS, int ACT>
__device__ __forceinline__ void store_direct16_k(const Args &p, const f32x16 (&acc)[TM][TN],
                                                 int r0, int c0, int lane) {
    using E = T16<BF>;
    static_assert(TN % 2 == 0, "block pairs");
    const int l32 = lane & 31, e = lane & 3, a4 = l32 & ~3, h = lane >> 5;
    const int rl = 4 * h + e;  // row within each group of 8, before the exchange
    auto pick = [](const f32x16 &a, int k) {
        f32x4 x;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            x[q] = k == 0 ? a[q] : k == 1 ? a[4 + q] : k == 2 ? a[8 + q] : a[12 + q];
        return x;
    };
#pragma unroll
    for (int jp = 0; jp < TN; jp += 2) {
        const int col0 = c0 + 32 * jp + a4, col1 = col0 + 32;
        const int colh = col0 + 32 * h;  // the block this lane stores
        f32x4 bv0 = {0.f, 0.f, 0.f, 0.f}, bv1 = bv0;
        if constexpr (MODE == 0 && BIAS) {
            bv0 = unpack4(BF, *reinterpret_cast<const u32x2 *>(p.bias + col0));
            bv1 = unpack4(BF, *reinterpret_cast<const u32x2 *>(p.bias + col1));
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const f32x16 &a0 = acc[i][jp], &a1 = acc[i][jp + 1];
            const int rowb = r0 + 32 * i + rl;
            constexpr bool kZs = MODE == 1 && ACT != kActNone;
            u32x2 zr0[4], zr1[4];
            if constexpr (kZs) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint16_t *zq = p.Zs + (size_t)(rowb + 8 * k) * p.ldzs;
                    zr0[k] = *reinterpret_cast<const u32x2 *>(zq + col0);
                    zr1[k] = *reinterpret_cast<const u32x2 *>(zq + col1);
                }
            }
#pragma unroll 1
            for (int k = 0; k < 4; ++k) {
                const f32x4 y0 = quad_transpose4(pick(a0, k), e);
                const f32x4 y1 = quad_transpose4(pick(a1, k), e);
                const int row = rowb + 8 * k;                     // this lane's row now
                const int rowA = r0 + 32 * i + 8 * k + e, rowB = rowA + 4;
                if constexpr (MODE == 2) {
                    *reinterpret_cast<f32x4 *>(p.partial + (size_t)row * p.N + col0) = y0;
                    *reinterpret_cast<f32x4 *>(p.partial + (size_t)row * p.N + col1) = y1;
                } else {
                    f32x4 z0 = {0.f, 0.f, 0.f, 0.f}, z1 = z0, o0 = z0, o1 = z0;
                    if constexpr (kZs) {
                        z0 = unpack4(BF, k == 0 ? zr0[0] : k == 1 ? zr0[1] : k == 2 ? zr0[2] : zr0[3]);
                        z1 = unpack4(BF, k == 0 ? zr1[0] : k == 1 ? zr1[1] : k == 2 ? zr1[2] : zr1[3]);
                    }
                    if (p.accumulate) {
                        const uint16_t *cq = p.C + (size_t)row * p.ldc;
                        o0 = unpack4(BF, *reinterpret_cast<const u32x2 *>(cq + col0));
                        o1 = unpack4(BF, *reinterpret_cast<const u32x2 *>(cq + col1));
                    }
                    u32x2 zp0, zp1;
                    const u32x2 c0v = epi16_x4_k<BF, MODE, BIAS, ACT>(p, y0, bv0, z0, o0, &zp0);
                    const u32x2 c1v = epi16_x4_k<BF, MODE, BIAS, ACT>(p, y1, bv1, z1, o1, &zp1);
                    auto xch = [&](u32x2 w0, u32x2 w1, uint16_t *base, int ld) {
                        const u32x2 send = h ? w0 : w1;
                        const u32x2 recv = {(uint32_t)__shfl_xor((int)send[0], 32),
                                            (uint32_t)__shfl_xor((int)send[1], 32)};
                        *reinterpret_cast<u32x2 *>(base + (size_t)rowA * ld + colh) = h ? recv : w0;
                        *reinterpret_cast<u32x2 *>(base + (size_t)rowB * ld + colh) = h ? w1 : recv;
                    };
                    if (MODE == 0 && p.Z) xch(zp0, zp1, p.Z, p.ldz);
                    xch(c0v, c1v, p.C, p.ldc);
                }
            }
        }
    }
}

// Picks the register epilogue's kind; an activation code outside ReLU / GELU
// takes the kind without one (the staged epilogue's act_fwd / act_grad are
// the identity for it, so the bits agree).
template <bool BF, int TM, int TN>
__device__ __forceinline__ void store_direct16(const Args &p, const f32x16 (&acc)[TM][TN], int r0,
                                               int c0, int lane) {
    if (p.ksplit > 0) {
        store_direct16_k<BF, TM, TN, 2, false, kActNone>(p, acc, r0, c0, lane);
    } else if (p.mode == 0) {
        if (p.bias) {
            if (p.act == kActRelu) store_direct16_k<BF, TM, TN, 0, true, kActRelu>(p, acc, r0, c0, lane);
            else if (p.act == kActGelu) store_direct16_k<BF, TM, TN, 0, true, kActGelu>(p, acc, r0, c0, lane);
            else store_direct16_k<BF, TM, TN, 0, true, kActNone>(p, acc, r0, c0, lane);
        } else {
            if (p.act == kActRelu) store_direct16_k<BF, TM, TN, 0, false, kActRelu>(p, acc, r0, c0, lane);
            else if (p.act == kActGelu) store_direct16_k<BF, TM, TN, 0, false, kActGelu>(p, acc, r0, c0, lane);
            else store_direct16_k<BF, TM, TN, 0, false, kActNone>(p, acc, r0, c0, lane);
        }
    } else {
        if (p.act == kActRelu) store_direct16_k<BF, TM, TN, 1, false, kActRelu>(p, acc, r0, c0, lane);
        else if (p.act == kActGelu) store_direct16_k<BF, TM, TN, 1, false, kActGelu>(p, acc, r0, c0, lane);
        else store_direct16_k<BF, TM, TN, 1, false, kActNone>(p, acc, r0, c0, lane);
    }
}

template <int BM, int BN, int BK, int WGM, int WGN, bool AK, bool BNC, bool VEC, bool BF>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm16_mfma(Args p) {
    using E = T16<BF>;
    constexpr int NT = 64 * WGM * WGN;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
    static_assert(BK % 16 == 0, "BK must be a multiple of 16");
    constexpr int kLd = BK + 8;
    constexpr int kASz = BM * kLd, kBSz = BN * kLd;  // elements
    constexpr int kBuf = kASz + kBSz;
    constexpr int kStageLd = WTN + 4;                 // floats
    constexpr int kStageBytes = WGM * WGN * 32 * kStageLd * 4;
    constexpr int kBytes = (4 * kBuf > kStageBytes) ? 4 * kBuf : kStageBytes;
    __shared__ __attribute__((aligned(16))) uint16_t lds[kBytes / 2];

    int tile_m, tile_n;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tile_m, tile_n);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // A is k-contiguous unless TN; B is k-contiguous only for NT.
    Loader<BM, BK, AK, VEC, NT> la;
    Loader<BN, BK, !BNC, VEC, NT> lb;
    const int nk = (p.K + BK - 1) / BK;

    la.load(p.A, p.lda, m0, p.M, 0, p.K);
    lb.load(p.B, p.ldb, n0, p.N, 0, p.K);
    la.store(lds);
    lb.store(lds + kASz);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            la.load(p.A, p.lda, m0, p.M, (kt + 1) * BK, p.K);
            lb.load(p.B, p.ldb, n0, p.N, (kt + 1) * BK, p.K);
        }
        const uint16_t *As = lds + cur * kBuf;
        const uint16_t *Bs = As + kASz;
#pragma unroll
        for (int u = 0; u < BK / 16; ++u) {
            const int kb = u * 16 + 8 * h;
            u32x4 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                a[i] = *reinterpret_cast<const u32x4 *>(As + (wm0 + i * 32 + l32) * kLd + kb);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[j] = *reinterpret_cast<const u32x4 *>(Bs + (wn0 + j * 32 + l32) * kLd + kb);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = E::mfma(a[i], b[j], acc[i][j]);
        }
        if (more) {
            uint16_t *nxt = lds + (cur ^ 1) * kBuf;
            la.store(nxt);
            lb.store(nxt + kASz);
        }
        __syncthreads();
    }

    store_tile16<BF, TM, TN, WTN, WGM * WGN>(p, acc, reinterpret_cast<float *>(lds), m0 + wm0,
                                             n0 + wn0, wave, lane);
}

// ------------------------------------------------ pipelined variant
// Software-pipelined over whole K tiles, one barrier per tile.  Each wave
// loads its share of a tile as 16 bytes (8 elements) per lane, lane l's
// chunk of wave load li landing at element 512 li + 8 l of the operand's
// stage area; the source of each chunk is chosen so that the stage ends up
// in the swizzled layout below.  Two ways to move the chunks:
//  * staged (BK 32 tiles but 256x256 with 4 waves): global loads into
//    registers, two register sets alternating by tile parity, written to a
//    two-stage LDS ring by ds_write_b128 one tile later;
//  * direct (BK 64 tiles, and 256x256 with 4 waves, whose accumulators leave
//    no room for two register sets): global_load_lds_dwordx4 (inline
//    assembly, lds_dma16) straight into an LDS ring of up to four stages,
//    as many as fit -- three for 256x128 tiles, whose two tiles in flight
//    ran their NT data gradient 917-922 -> 944-948 TF at 2048x4096x4096
//    (bf16 c5 step 2.066-2.070 -> 2.037-2.042 ms).
// A BK of 32 or 64 is only 1-2 thousand MFMA cycles per SIMD, so the barrier
// is overlapped: the last k16 step of each tile is multiplied after it, from
// registers.  No operand is transposed on its way in:
//  * a k-contiguous operand sits [rows][BK]; chunk c (8 k) of row r at
//    c ^ ((r / (128 / BK)) % (BK / 8)), so the rows read together by a
//    16-byte LDS read hit distinct banks; an MFMA operand is one such read;
//  * a row-contiguous operand sits [BK][R] as loaded; chunk c of k-row k at
//    c ^ (4 * (k % 4)).  Its MFMA operand (8 consecutive k of one row) comes
//    from two ds_read_b64_tr_b16: within each 16-lane group, source lane
//    4e + q reads the 4 elements at (k0 + e, r0 + 4q .. + 3) and output lane
//    l receives (k0 + 0..3, r0 + l) -- the layout measured on gfx950 with an
//    in-bounds probe; the swizzle keeps the group's 4 k-rows on distinct banks.
// Used when K % BK == 0, leading dimensions are multiples of 8 with 16-byte
// aligned bases, and each row-contiguous operand's row length is a multiple
// of 8 (edge chunks are clamped to the last valid one; they reach only
// masked outputs).
typedef short v4i16 __attribute__((ext_vector_type(4)));

template <int BK>
__device__ __forceinline__ int swz16_k(int row) {
    return (row / (128 / BK)) % (BK / 8);
}
__device__ __forceinline__ int swz16_r(int k) { return 4 * (k & 3); }

// 8 consecutive k (k0 .. k0+7, k0 a multiple of 8) of row `row` of a
// row-contiguous [BK][R] tile, as one MFMA operand: two transposing reads.
template <int R>
__device__ __forceinline__ u32x4 read_tr(const uint16_t *tile, int k0, int row_base, int lane) {
    const int i = lane & 15;             // source lane within the 16-lane group
    const int e = i >> 2, q = i & 3;
    const int r = row_base + 4 * q;      // first of the 4 elements this lane reads
    u32x4 out;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int k = k0 + 4 * half + e;
        const int idx = k * R + ((((r >> 3) ^ swz16_r(k)) << 3) | (r & 7));
        const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16 *)(tile + idx));
        const u32x2 w = __builtin_bit_cast(u32x2, v);
        out[2 * half] = w[0];
        out[2 * half + 1] = w[1];
    }
    return out;
}

// Column sums of the B tiles of the TN layout (B row-contiguous, [BK][BN]
// in LDS with chunk c of k-row k at chunk c ^ swz16_r(k)), for the bias
// gradient, taken by the workgroups of tile row 0: thread t owns the 8
// columns of chunk t % (BN / 8) and k-rows (t / (BN / 8)) * KPT .. + KPT of
// each tile, summed in fp32; the k-groups are added in a fixed order at the
// end (deterministic).
template <int BN, int BK, int NT, bool BF>
struct ColSum16 {
    static constexpr int kChunks = BN / 8;
    static constexpr int G = NT / kChunks;  // k-groups
    static constexpr int KPT = BK / G;      // k-rows per thread and tile
    static_assert(NT % kChunks == 0 && BK % G == 0 && KPT >= 1, "column-sum split");
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

    __device__ __forceinline__ void add(const uint16_t *Bs) {
        const int c = threadIdx.x % kChunks, g = threadIdx.x / kChunks;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int k = g * KPT + i;
            const u32x4 w =
                *reinterpret_cast<const u32x4 *>(Bs + k * BN + ((c ^ swz16_r(k)) << 3));
#pragma unroll
            for (int e = 0; e < 8; ++e)
                s[e] += T16<BF>::to_f((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
        }
    }
    // The rows k0 .. K-1 past the whole tiles (fewer than BK), from global
    // memory in the same thread-to-(column, k-row) assignment, after the
    // tiles' rows.
    __device__ __forceinline__ void add_tail(const uint16_t *B, int ldb, int k0, int K, int n0,
                                             int N) {
        const int c = threadIdx.x % kChunks, g = threadIdx.x / kChunks;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int k = k0 + g * KPT + i;
            if (k >= K) continue;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                s[e] += T16<BF>::to_f(B[(size_t)k * ldb + min(n0 + c * 8 + e, N - 1)]);
        }
    }
    // Combines the k-groups through lds (G * BN floats, free) and writes the
    // tile's columns.  Called by every thread of the workgroup.
    __device__ __forceinline__ void finish(const Args &p, float *lds, int n0) const {
        const int c = threadIdx.x % kChunks, g = threadIdx.x / kChunks;
#pragma unroll
        for (int e = 0; e < 8; ++e) lds[g * BN + c * 8 + e] = s[e];
        __syncthreads();
        for (int col = threadIdx.x; col < BN; col += NT) {
            if (n0 + col >= p.N) continue;
            float t = 0.0f;
#pragma unroll
            for (int k = 0; k < G; ++k) t += lds[k * BN + col];
            if (p.ksplit > 0) {  // a K slice: its fp32 sums, finished by sum_slices16
                p.colsum_partial[n0 + col] = t;
                continue;
            }
            uint16_t *dst = p.colsum + n0 + col;
            *dst = T16<BF>::from_f(p.colsum_accumulate ? T16<BF>::to_f(*dst) + t : t);
        }
        __syncthreads();
    }
};

// LDS of the pipelined kernel, in 16-bit elements: its stages (staged
// loads -- global -> registers -> ds_write -- for BK 32 tiles but 256x256
// with 4 waves (256 accumulator registers): two; direct-to-LDS loads: up to
// four, as many as fit in the 160 KiB of LDS) or the epilogue's fp32
// staging, whichever is larger.
template <int BM, int BN, int BK, int WGM, int WGN>
struct Pipe16Lds {
    static constexpr int kNW = WGM * WGN;
    static constexpr int kStageSz = BM * BK + BN * BK;  // elements
    static constexpr bool kStaged = BK == 32 && !(BM == 256 && BN == 256 && kNW == 4);
    static constexpr int kStages = kStaged                             ? 2
                                   : 4 * kStageSz * 2 <= 160 * 1024   ? 4
                                   : 3 * kStageSz * 2 <= 160 * 1024 ? 3
                                                                     : 2;
    static constexpr int kEpiBytes = kNW * 32 * (BN / WGN + 4) * 4;
    static constexpr int kBytes =
        (kStages * kStageSz * 2 > kEpiBytes) ? kStages * kStageSz * 2 : kEpiBytes;
    static constexpr int elems = kBytes / 2;
};

// The kernel's LDS buffer of N 16-bit elements: one static array per N, so
// bodies that ask for the same N in one launch share it.
template <int N>
__device__ __forceinline__ uint16_t (&lds16_buffer())[N] {
    __shared__ __attribute__((aligned(16))) uint16_t buf[N];
    return buf;
}

// The pipelined 16-bit GEMM for output tile bx (and K slice by when split).
// LDSN: the LDS buffer's size in elements, at least Pipe16Lds::elems (0:
// just that) -- a launch running several bodies gives them all the largest.
// KT: K need not be a multiple of BK (K % 8 == 0 where an operand is
// k-contiguous): the tile loop runs the whole tiles, and the k past them go
// into the accumulators from global memory at the end (the K tail below).
template <int BM, int BN, int BK, int WGM, int WGN, bool AK, bool BNC, bool BF, int LDSN = 0,
          bool KT = false>
__device__ __forceinline__ void gemm16_pipe_body(Args p, int bx, int by) {
    using E = T16<BF>;
    constexpr int NW = WGM * WGN;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
    static_assert(BK == 32 || BK == 64, "BK 32 or 64");
    static_assert(BM >= 128 && BN >= 128, "row-contiguous tiles need >= 16 chunks per k-row");
    constexpr int kInstA = BM * BK / 8 / 64, kInstB = BN * BK / 8 / 64;
    static_assert(kInstA % NW == 0 && kInstB % NW == 0, "loads divide among the waves");
    constexpr int kPerA = kInstA / NW, kPerB = kInstB / NW, kLoads = kPerA + kPerB;
    constexpr int kASz = BM * BK, kBSz = BN * BK, kStageSz = kASz + kBSz;  // elements
    using PL = Pipe16Lds<BM, BN, BK, WGM, WGN>;
    constexpr bool kStaged = PL::kStaged;
    constexpr int kStages = PL::kStages;
    static_assert(LDSN == 0 || LDSN >= PL::elems, "LDS buffer too small");
    uint16_t(&lds)[LDSN ? LDSN : PL::elems] = lds16_buffer<LDSN ? LDSN : PL::elems>();

    if (p.ksplit > 0) {  // K slice by: offset operands, its own slot
        const int kb = by * p.ksplit;
        p.A += AK ? (size_t)kb : (size_t)kb * p.lda;
        p.B += BNC ? (size_t)kb * p.ldb : (size_t)kb;
        p.K = min(p.ksplit, p.K - kb);
        p.partial += (size_t)by * p.M * p.N;
        if (p.colsum) p.colsum_partial += (size_t)by * p.N;
    }
    int tile_m, tile_n;
    tile_of(bx, p.tiles_m, p.tiles_n, tile_m, tile_n);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    // The wave index, as a uniform (scalar) value: it selects LDS destinations
    // and operands per wave, which the compiler would otherwise treat as
    // varying across lanes.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto src_kc = [&](const uint16_t *base, int ld, int r0, int rmax, int k0, int pos) {
        const int row = pos / (BK / 8), pc = pos % (BK / 8);
        const int c = pc ^ swz16_k<BK>(row);
        return base + (size_t)min(r0 + row, rmax - 1) * ld + k0 + 8 * c;
    };
    auto src_rc = [&](const uint16_t *base, int ld, int r0, int rmax, int k0, int pos, int R) {
        const int k = pos / (R / 8), pc = pos % (R / 8);
        const int c = pc ^ swz16_r(k);
        return base + (size_t)(k0 + k) * ld + min(r0 + 8 * c, rmax - 8);
    };
    // Wave load q (0 .. kLoads-1) of tile kt into stage `stage`: this wave's
    // share of A first, then of B.
    auto issue_one = [&](int kt, int stage, int q) {
        uint16_t *sa = lds + stage * kStageSz;
        const int k0 = kt * BK;
        if (q < kPerA) {
            const int li = wave * kPerA + q, pos = li * 64 + lane;
            const uint16_t *src = AK ? src_kc(p.A, p.lda, m0, p.M, k0, pos)
                                     : src_rc(p.A, p.lda, m0, p.M, k0, pos, BM);
            lds_dma16(src, sa + li * 512);
        } else {
            const int li = wave * kPerB + (q - kPerA), pos = li * 64 + lane;
            const uint16_t *src = BNC ? src_rc(p.B, p.ldb, n0, p.N, k0, pos, BN)
                                      : src_kc(p.B, p.ldb, n0, p.N, k0, pos);
            lds_dma16(src, sa + kASz + li * 512);
        }
    };
    auto issue = [&](int kt, int stage) {
#pragma unroll
        for (int q = 0; q < kLoads; ++q) issue_one(kt, stage, q);
    };
    // Staged: wave load q of tile kt into registers, and from there to its
    // place in a stage (lane l's 16 bytes at element 8 l of the wave load's
    // 1 KiB run, as the direct loads would put them).
    auto load_reg = [&](int kt, int q) {
        const int k0 = kt * BK;
        const uint16_t *src;
        if (q < kPerA) {
            const int pos = (wave * kPerA + q) * 64 + lane;
            src = AK ? src_kc(p.A, p.lda, m0, p.M, k0, pos) : src_rc(p.A, p.lda, m0, p.M, k0, pos, BM);
        } else {
            const int pos = (wave * kPerB + (q - kPerA)) * 64 + lane;
            src = BNC ? src_rc(p.B, p.ldb, n0, p.N, k0, pos, BN) : src_kc(p.B, p.ldb, n0, p.N, k0, pos);
        }
        return *reinterpret_cast<const u32x4 *>(src);
    };
    auto store_reg = [&](int stage, int q, const u32x4 &v) {
        uint16_t *sa = lds + stage * kStageSz;
        uint16_t *run = q < kPerA ? sa + (wave * kPerA + q) * 512
                                  : sa + kASz + (wave * kPerB + q - kPerA) * 512;
        *reinterpret_cast<u32x4 *>(run + 8 * lane) = v;
    };

    const int nk = p.K / BK;
    constexpr bool kTN = !AK && BNC;
    ColSum16<BN, BK, 64 * NW, BF> cs;
    const bool do_cs = kTN && p.colsum && tile_m == 0;
    // MFMA operands of k16 step u of a stage: lane half h takes k 8h .. 8h+7.
    auto frag_a = [&](const uint16_t *As, int u, int i) {
        const int kb = u * 16 + 8 * h;
        if constexpr (AK) {
            const int row = wm0 + i * 32 + l32;
            const int c = (kb >> 3) ^ swz16_k<BK>(row);
            return *reinterpret_cast<const u32x4 *>(As + row * BK + 8 * c);
        } else {
            return read_tr<BM>(As, kb, wm0 + i * 32 + 16 * ((lane >> 4) & 1), lane);
        }
    };
    auto frag_b = [&](const uint16_t *Bs, int u, int j) {
        const int kb = u * 16 + 8 * h;
        if constexpr (BNC) {
            return read_tr<BN>(Bs, kb, wn0 + j * 32 + 16 * ((lane >> 4) & 1), lane);
        } else {
            const int col = wn0 + j * 32 + l32;
            const int c = (kb >> 3) ^ swz16_k<BK>(col);
            return *reinterpret_cast<const u32x4 *>(Bs + col * BK + 8 * c);
        }
    };
    auto frag = [&](const uint16_t *As, const uint16_t *Bs, int u, u32x4 (&a)[TM], u32x4 (&b)[TN]) {
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = frag_a(As, u, i);
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = frag_b(Bs, u, j);
    };
    constexpr int NU = BK / 16;
    constexpr int kMfma = TM * TN;                       // MFMAs per k16 step
    constexpr int kPieces = TM + TN;                     // operand fragments per step
    constexpr int kSlots = (NU - 1) * kMfma;             // MFMAs of a tile before its barrier
    static_assert(NU >= 2 && kLoads <= kSlots, "a tile's loads fit among its MFMAs");
    // MFMAs per load: staged, spread over the steps before the barrier;
    // direct, one per MFMA from the tile's first step, which leaves them
    // most of the tile to land (the two-stage ring of the 256x256 tiles
    // waits for them at the tile's end): 4096^3 NN / NT / TN 1160-1167 /
    // 1166-1178 / 1127-1149 -> 1202-1210 / 1215-1226 / 1186-1196 TF, the
    // 256x128 tiles of the c5 shapes unchanged.  Issuing them a step
    // earlier still, among the MFMAs right after the barrier that frees
    // their stage, measured 1181 / 1191 / 1162.
    constexpr int kStride = kStaged ? kSlots / kLoads : 1;
    constexpr int kAhead = kStages - 1;                  // direct: tiles in flight
    // One k16 step's MFMAs on (ca, cb) in a fixed order: after MFMA m, the
    // reads of operand fragment m of step un (A fragments, then B), and, when
    // `ld`, the tile's memory operations that fall on this step's slots (one
    // every kStride MFMAs over the steps before the tile's barrier): staged,
    // register set Rw's chunk q (tile kt+1) written to stage `slot` and the
    // register refilled from tile kl (Rl); direct, one load of tile kl into
    // stage `slot`.  Reads or loads issued in a burst fill the wave's memory
    // queues and hold up the MFMAs behind them.
    auto run_step = [&](const u32x4 (&ca)[TM], const u32x4 (&cb)[TN], const uint16_t *An,
                        const uint16_t *Bn, int un, u32x4 (&na)[TM], u32x4 (&nb)[TN], int u,
                        bool ld, int kl, int slot, const u32x4 *Rw, u32x4 *Rl) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < (kMfma > kPieces ? kMfma : kPieces); ++m) {
            if (m < kMfma) {
                const int i = m / TN, j = m % TN;
                acc[i][j] = E::mfma(ca[i], cb[j], acc[i][j]);
            }
            if (m < TM)
                na[m] = frag_a(An, un, m);
            else if (m < kPieces)
                nb[m - TM] = frag_b(Bn, un, m - TM);
            if (ld && m < kMfma) {
                const int sidx = u * kMfma + m;
                if (sidx % kStride == 0 && sidx / kStride < kLoads) {
                    const int q = sidx / kStride;
                    if constexpr (kStaged) {
                        store_reg(slot, q, Rw[q]);
                        Rl[q] = load_reg(kl, q);
                    } else {
                        issue_one(kl, slot, q);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Barrier-overlapped loop: the last k16 step of tile kt is read into
    // registers before the barrier that ends tile kt and multiplied after
    // it, so the matrix units stay busy across the barrier while the first
    // operands of tile kt+1 are read.  Tile t lives in stage t % kStages.
    // Operands are double-buffered in registers: the reads of step u+1 go
    // out among the MFMAs of step u; ca / cb hold the operands of the next
    // step to multiply.
    u32x4 ca[TM], cb[TN];
    auto tile = [&](int kt, int kl, int slot, const u32x4 *Rw, u32x4 *Rl) {
        const uint16_t *As = lds + (kt % kStages) * kStageSz;
        const uint16_t *Bs = As + kASz;
#pragma unroll
        for (int u = 0; u < NU - 1; ++u) {
            // Step u's operands (read during the previous step) have landed;
            // waiting here, before the next step's reads are issued, leaves
            // those in flight behind the MFMAs.
            wait_lgkm0();
            u32x4 na[TM], nb[TN];
            run_step(ca, cb, As, Bs, u + 1, na, nb, u, true, kl, slot, Rw, Rl);
#pragma unroll
            for (int i = 0; i < TM; ++i) ca[i] = na[i];
#pragma unroll
            for (int j = 0; j < TN; ++j) cb[j] = nb[j];
        }
        if constexpr (kTN)
            if (do_cs) cs.add(Bs);
        // ca / cb: the last step of tile kt.  Every wave's reads (and LDS
        // writes) of this tile are done before the barrier; direct, this
        // wave's loads of tile kt+1 are done once at most the newest
        // kAhead-1 tiles' are outstanding, and the barrier publishes every
        // wave's.
        wait_lgkm0();
        if constexpr (!kStaged) wait_vmcnt<(kAhead - 1) * kLoads>();
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_barrier" ::: "memory");
        // Step 0 of tile kt+1 (past the last tile: a stage nothing uses,
        // read and discarded).
        u32x4 na[TM], nb[TN];
        const uint16_t *An = lds + ((kt + 1) % kStages) * kStageSz;
        run_step(ca, cb, An, An + kASz, 0, na, nb, 0, false, 0, 0, Rw, Rl);
#pragma unroll
        for (int i = 0; i < TM; ++i) ca[i] = na[i];
#pragma unroll
        for (int j = 0; j < TN; ++j) cb[j] = nb[j];
    };
    if constexpr (kStaged) {
        // Tile t is loaded into register set t % 2 during tile t-2 and
        // written from there to stage t % 2 during tile t-1 (the stage of
        // tile t-2, free since the barrier that ended tile t-2); each write
        // goes out right before the load that refills its registers.  Past
        // the last tile, tile nk-1 is reloaded and written to the free
        // stage, which nothing reads.  The kt loop is unrolled by two so
        // that the register sets swap roles without copies.
        if (nk > 0) {
            u32x4 R0[kLoads], R1[kLoads];
#pragma unroll
            for (int q = 0; q < kLoads; ++q) R0[q] = load_reg(0, q);
#pragma unroll
            for (int q = 0; q < kLoads; ++q) R1[q] = load_reg(min(1, nk - 1), q);
#pragma unroll
            for (int q = 0; q < kLoads; ++q) store_reg(0, q, R0[q]);
            wait_lgkm0();
            asm volatile("s_barrier" ::: "memory");
            frag(lds, lds + kASz, 0, ca, cb);
            // Tile kt writes the set holding tile kt+1 and refills the other
            // with tile kt+2; that set was loaded a whole tile ago.
            int kt = 0;
            for (; kt + 1 < nk; kt += 2) {
                wait_vmcnt<0>();
                tile(kt, min(kt + 2, nk - 1), (kt + 1) % kStages, R1, R0);
                wait_vmcnt<0>();
                tile(kt + 1, min(kt + 3, nk - 1), kt % kStages, R0, R1);
            }
            if (kt < nk) {
                wait_vmcnt<0>();
                tile(kt, nk - 1, (kt + 1) % kStages, R1, R0);
            }
        }
    } else {
        // Tile t goes to stage t % kStages.  The prologue issues tiles
        // 0 .. kAhead-1; iteration kt issues tile kt + kAhead into the stage
        // of tile kt-1, free since the barrier that ended tile kt-1.  Past
        // the last tile an iteration reloads tile nk-1 into that free stage,
        // which nothing reads again: the loop body has no branch, and every
        // iteration leaves the same kAhead tiles in flight.
        if (nk > 0) {
#pragma unroll
            for (int t = 0; t < kAhead; ++t) issue(min(t, nk - 1), t);
            wait_vmcnt<(kAhead - 1) * kLoads>();  // tile 0 landed
            asm volatile("s_barrier" ::: "memory");
            frag(lds, lds + kASz, 0, ca, cb);
            for (int kt = 0; kt < nk; ++kt)
                tile(kt, min(kt + kAhead, nk - 1), (kt + kAhead) % kStages, nullptr, nullptr);
            wait_vmcnt<0>();  // the reloads past the last tile, before the LDS reuse
        }
    }
    // K tail (KT): k = kb .. K-1 past the whole tiles, in k16 steps as a tile
    // takes them (lane half h supplies k = kb + 16 s + 8 h .. + 7 of its row /
    // column), zeros for a lane's k past K and the steps entirely past K
    // skipped.  A lane takes its eight k of a k-contiguous operand with one
    // 16-byte load (K % 8 == 0 there), of a row-contiguous one with eight
    // loads coalesced across the lanes; every address is clamped into the
    // operand, and all loads go out before the first MFMA.  The column sums
    // (TN) add the same k after the tiles'.
    if constexpr (KT) {
        const int kb = nk * BK;
        if (kb < p.K) {
            constexpr int NS = BK / 16;
            int arow[TM], bcol[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) arow[i] = min(m0 + wm0 + 32 * i + l32, p.M - 1);
#pragma unroll
            for (int j = 0; j < TN; ++j) bcol[j] = min(n0 + wn0 + 32 * j + l32, p.N - 1);
            auto eight = [&](const uint16_t *base, int ld, bool kc, int r, int k8) {
                u32x4 v;
                if (kc) {
                    v = *reinterpret_cast<const u32x4 *>(base + (size_t)r * ld + min(k8, p.K - 8));
                    if (k8 >= p.K) v = u32x4{0u, 0u, 0u, 0u};
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const uint16_t x = base[(size_t)min(k8 + t, p.K - 1) * ld + r];
                        e[t] = k8 + t < p.K ? x : (uint16_t)0;
                    }
                    v = u32x4{pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]),
                              pack2(e[6], e[7])};
                }
                return v;
            };
            u32x4 ta[NS][TM], tb[NS][TN];
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                if (kb + 16 * st >= p.K) continue;  // uniform
                const int k8 = kb + 16 * st + 8 * h;
#pragma unroll
                for (int i = 0; i < TM; ++i) ta[st][i] = eight(p.A, p.lda, AK, arow[i], k8);
#pragma unroll
                for (int j = 0; j < TN; ++j) tb[st][j] = eight(p.B, p.ldb, !BNC, bcol[j], k8);
            }
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                if (kb + 16 * st >= p.K) continue;
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = E::mfma(ta[st][i], tb[st][j], acc[i][j]);
            }
            if constexpr (kTN)
                if (do_cs) cs.add_tail(p.B, p.ldb, kb, p.K, n0, p.N);
        }
    }
    __syncthreads();
    if constexpr (kTN)
        if (do_cs) cs.finish(p, reinterpret_cast<float *>(lds), n0);
    // The whole tile in bounds: the register epilogue (uniform across the
    // workgroup, as the staged one has workgroup barriers).
    // It pairs blocks, so it needs an even TN (the 64x64 tile keeps the
    // staged one); waves holding 256 accumulator registers (the 4-wave
    // 256x256 tiles) keep it too, as the register epilogue's temporaries
    // would spill there.
    constexpr bool kDirect = TN % 2 == 0 && TM * TN <= 8;
    bool direct = false;
    if constexpr (kDirect)
        direct = p.vec_out && m0 + BM <= p.M && n0 + BN <= p.N && (p.ksplit == 0 || p.N % 4 == 0);
    if (direct) {
        if constexpr (kDirect) store_direct16<BF, TM, TN>(p, acc, m0 + wm0, n0 + wn0, lane);
    } else {
        store_tile16<BF, TM, TN, WTN, NW>(p, acc, reinterpret_cast<float *>(lds), m0 + wm0,
                                          n0 + wn0, wave, lane);
    }
}

template <int BM, int BN, int BK, int WGM, int WGN, bool AK, bool BNC, bool BF, bool KT = false>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm16_pipe(Args p) {
    gemm16_pipe_body<BM, BN, BK, WGM, WGN, AK, BNC, BF, 0, KT>(p, blockIdx.x, blockIdx.y);
}

// A large layer's weight gradient (TN, 256x256 tiles, 8 waves, BK 64, direct
// loads: workgroups below n1) and data gradient (NT, 256x128 tiles, 8 waves, BK
// 64, direct loads: the rest) in one launch, each body exactly as its own kernel, both on
// one LDS buffer of the larger size: the dW tiles' output writes drain while
// dX tiles compute, where two launches would leave the CUs idle through them.
constexpr int kPair16Lds = Pipe16Lds<256, 256, 64, 2, 4>::elems > Pipe16Lds<256, 128, 64, 4, 2>::elems
                               ? Pipe16Lds<256, 256, 64, 2, 4>::elems
                               : Pipe16Lds<256, 128, 64, 4, 2>::elems;
template <bool BF>
__global__ __launch_bounds__(512) void gemm16_pair_big(Args a1, Args a2, int n1) {
    const int w = blockIdx.x;
    if (w < n1)
        gemm16_pipe_body<256, 256, 64, 2, 4, false, true, BF, kPair16Lds>(a1, w, 0);
    else
        gemm16_pipe_body<256, 128, 64, 4, 2, true, false, BF, kPair16Lds>(a2, w - n1, 0);
}
template <bool BF>
void launch_pair16(Args a1, Args a2, hipStream_t st) {
    a1.tiles_m = (a1.M + 255) / 256;
    a1.tiles_n = (a1.N + 255) / 256;
    a2.tiles_m = (a2.M + 255) / 256;
    a2.tiles_n = (a2.N + 127) / 128;
    const int n1 = a1.tiles_m * a1.tiles_n, n2 = a2.tiles_m * a2.tiles_n;
    gemm16_pair_big<BF><<<n1 + n2, 512, 0, st>>>(a1, a2, n1);
}
// The pair's configurations (see launch_layout): dW on cfg 6, dX on cfg 8.
constexpr int kPair16CfgW = 6, kPair16CfgX = 8;

// The slots of a K-split GEMM summed in slot order (fp32), then the GEMM's
// epilogue applied to each sum exactly as the kernel applies it to its own
// (epi16_x4 on four columns, epi16 on the last few of a row).  One thread
// per four columns of a row.
template <bool BF>
__global__ __launch_bounds__(256) void sum_slices16(Args p, int splits) {
    using E = T16<BF>;
    const int g4 = (p.N + 3) / 4;
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= (int64_t)p.M * g4) return;
    const int row = (int)(q / g4), col = (int)(q % g4) * 4;
    const size_t slot = (size_t)p.M * p.N;
    if (row == 0 && p.colsum) {  // the column sums' slots, in slot order
#pragma unroll 1
        for (int t = 0; t < 4 && col + t < p.N; ++t) {
            float v = p.colsum_partial[col + t];
#pragma unroll 1
            for (int s = 1; s < splits; ++s) v += p.colsum_partial[(size_t)s * p.N + col + t];
            uint16_t *dst = p.colsum + col + t;
            *dst = E::from_f(p.colsum_accumulate ? E::to_f(*dst) + v : v);
        }
    }
    const float *src = p.partial + (size_t)row * p.N + col;
    if (p.vec_out && p.N % 4 == 0) {
        f32x4 v = *reinterpret_cast<const f32x4 *>(src);
#pragma unroll 1
        for (int s = 1; s < splits; ++s) v += *reinterpret_cast<const f32x4 *>(src + s * slot);
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if (p.mode == 0 && p.bias) {
            const u32x2 w = *reinterpret_cast<const u32x2 *>(p.bias + col);
            bv = f32x4{E::to_f((uint16_t)w[0]), E::to_f((uint16_t)(w[0] >> 16)),
                       E::to_f((uint16_t)w[1]), E::to_f((uint16_t)(w[1] >> 16))};
        }
        epi16_x4<BF>(p, v, bv, row, col);
        return;
    }
    uint16_t *crow = p.C + (size_t)row * p.ldc;
    const uint16_t *bias = p.mode == 0 ? p.bias : nullptr;
#pragma unroll 1
    for (int t = 0; t < 4 && col + t < p.N; ++t) {
        float v = src[t];
#pragma unroll 1
        for (int s = 1; s < splits; ++s) v += src[t + s * slot];
        float zt;
        float ot = epi16<BF>(p, v, bias, row, col + t, &zt);
        if (p.mode == 0 && p.Z) p.Z[(size_t)row * p.ldz + col + t] = E::from_f(zt);
        if (p.accumulate) ot += E::to_f(crow[col + t]);
        crow[col + t] = E::from_f(ot);
    }
}

template <int BM, int BN, int WGM, int WGN, int BK, bool AK, bool BNC, bool BF, bool KT = false>
void launch_pipe16(const Args &a0, hipStream_t st) {
    Args a = a0;
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    const int splits = a.ksplit > 0 ? (a.K + a.ksplit - 1) / a.ksplit : 1;
    gemm16_pipe<BM, BN, BK, WGM, WGN, AK, BNC, BF, KT>
        <<<dim3(a.tiles_m * a.tiles_n, splits), 64 * WGM * WGN, 0, st>>>(a);
    if (splits > 1) {
        const int64_t threads = (int64_t)a.M * ((a.N + 3) / 4);
        sum_slices16<BF><<<(unsigned)((threads + 255) / 256), 256, 0, st>>>(a, splits);
    }
}

template <int BM, int BN, int WGM, int WGN, int BK, bool AK, bool BNC, bool VEC, bool BF>
void launch_one(const Args &a0, hipStream_t st) {
    Args a = a0;
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    gemm16_mfma<BM, BN, BK, WGM, WGN, AK, BNC, VEC, BF>
        <<<a.tiles_m * a.tiles_n, 64 * WGM * WGN, 0, st>>>(a);
}

// Tile configurations (BM x BN, waves, K depth):
//   0: 256x256, 4 waves, BK 32     1: 256x256, 8 waves, BK 32
//   2: 128x128, 4 waves, BK 32     3:  64x64,  4 waves, BK 32
//   4: 256x128, 4 waves, BK 32     5: 256x256, 4 waves, BK 64
//   6: 256x256, 8 waves, BK 64     7: 256x128, 4 waves, BK 64
//   8: 256x128, 8 waves, BK 64      9: 8's tiles with a K tail (K % 64 != 0)
// 64x64 is also the only element-load variant, for unaligned operands.
constexpr int kNumCfgs = 10;
constexpr int kCfgKTail16 = 9;

// K depth of a configuration.
inline int cfg_bk16(int cfg) { return cfg >= 5 ? 64 : 32; }

template <bool AK, bool BNC, bool BF>
void launch_layout(const Args &a, bool vec, bool pipe, int cfg, hipStream_t st) {
    if (!vec) {
        launch_one<64, 64, 2, 2, 32, AK, BNC, false, BF>(a, st);
        return;
    }
    if (pipe && cfg != 3) {
        switch (cfg) {
            case 0: launch_pipe16<256, 256, 2, 2, 32, AK, BNC, BF>(a, st); break;
            case 1: launch_pipe16<256, 256, 2, 4, 32, AK, BNC, BF>(a, st); break;
            case 2: launch_pipe16<128, 128, 2, 2, 32, AK, BNC, BF>(a, st); break;
            case 4: launch_pipe16<256, 128, 2, 2, 32, AK, BNC, BF>(a, st); break;
            case 5: launch_pipe16<256, 256, 2, 2, 64, AK, BNC, BF>(a, st); break;
            case 6: launch_pipe16<256, 256, 2, 4, 64, AK, BNC, BF>(a, st); break;
            case 7: launch_pipe16<256, 128, 2, 2, 64, AK, BNC, BF>(a, st); break;
            case kCfgKTail16: launch_pipe16<256, 128, 4, 2, 64, AK, BNC, BF, true>(a, st); break;
            default: launch_pipe16<256, 128, 4, 2, 64, AK, BNC, BF>(a, st); break;
        }
        return;
    }
    switch (cfg) {
        case 0: launch_one<256, 256, 2, 2, 32, AK, BNC, true, BF>(a, st); break;
        case 1: launch_one<256, 256, 2, 4, 32, AK, BNC, true, BF>(a, st); break;
        case 2: launch_one<128, 128, 2, 2, 32, AK, BNC, true, BF>(a, st); break;
        case 4: launch_one<256, 128, 2, 2, 32, AK, BNC, true, BF>(a, st); break;
        case 5: launch_one<256, 256, 2, 2, 64, AK, BNC, true, BF>(a, st); break;
        case 6: launch_one<256, 256, 2, 4, 64, AK, BNC, true, BF>(a, st); break;
        case 7: launch_one<256, 128, 2, 2, 64, AK, BNC, true, BF>(a, st); break;
        case 8:
        case kCfgKTail16: launch_one<256, 128, 4, 2, 64, AK, BNC, true, BF>(a, st); break;
        default: launch_one<64, 64, 2, 2, 32, AK, BNC, true, BF>(a, st); break;
    }
}

// Defined in k_gemm16_{bf16,f16}.hip.  layout: FG_NN / FG_NT / FG_TN.
void launch_bf16(int layout, const Args &a, bool vec, bool pipe, int cfg, hipStream_t st);
void launch_f16(int layout, const Args &a, bool vec, bool pipe, int cfg, hipStream_t st);
// gemm16_pair_big: dW (TN, a1) and dX (NT, a2), both planned pipelined on
// kPair16CfgW / kPair16CfgX without a K split.
void launch_pair_bf16(const Args &a1, const Args &a2, hipStream_t st);
void launch_pair_f16(const Args &a1, const Args &a2, hipStream_t st);

}  // namespace gemm16
}  // namespace fg
