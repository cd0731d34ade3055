// fg_gemm_kernel.h -- fp32 GEMM on CDNA4 matrix cores
// (v_mfma_f32_32x32x2_f32) with fused epilogues.  Included by the
// per-layout instantiation units k_gemm_{nn,nt,tn}.hip.
//
// Replaces the reference's matmul kernels: a 16x16 LDS tile per 256-thread
// block with one scalar fmaf per LDS pair (crates/ferrograd-nn/src/op/matmul/
// generic.rs:98-319), forward plus the dA / dB backward forms
// (op/matmul/mod.rs:75-125), and the elementwise producers/consumers the
// lowering inlines around them (kernel/forward.rs:298-464).
//
// Design (gfx950, 256 CUs, 64-wide waves, 160 KiB LDS per CU):
//  * 4 or 8 waves per workgroup; each wave owns a (TM*32)x(TN*32) block of
//    C held in TM*TN 16-register MFMA accumulators (up to 256 registers,
//    which the compiler places in AGPRs).
//  * K is consumed in BK-deep tiles (16 or 32) staged through LDS.  Where
//    whole K tiles and 16-byte alignment allow, gemm_f32_pipe runs a
//    software pipeline over them (loads two tiles ahead, fragments
//    double-buffered in registers, a fixed MFMA / LDS-read / load order,
//    swizzled unpadded layout); otherwise gemm_f32_mfma stages them through
//    registers into double-buffered LDS (the loads of tile t+1 in flight
//    during the MFMAs of tile t).  One barrier per tile either way.
//  * No operand is transposed on its way to LDS.  A k-contiguous operand is
//    kept [row][k] (row stride BK+4 floats, conflict-free 16-byte reads) and
//    a row-contiguous one [k][row] (stride rows+4).  The MFMA's k index is
//    permuted consistently for both operands so that a lane of a
//    k-contiguous operand reads 4 consecutive k with one ds_read_b128: in a
//    16-k tile, lane half h (lanes 32h..32h+31) feeds k = 8h + 4q + s to the
//    s-th MFMA of quad q.  Summation order inside the MFMA is hardware
//    defined; results match the CPU restatement within the 1e-5*sqrt(K)
//    tolerance, not bit for bit.
//  * The epilogue stages each wave's accumulators through LDS one 32-row
//    slice at a time and applies bias / activation / activation-derivative
//    on float4 groups, so global stores (and the reads of bias, Z) are
//    16-byte and coalesced.
//  * Workgroup ids are remapped so that the 8 XCDs (each with its own L2)
//    get contiguous groups of output tiles.
//  * Edge tiles are zero-filled on load and masked on store, so any M, N, K
//    work (the reference requires multiples of 16; N = 10 and N = 1000 of
//    the target configurations are not).
#pragma once

#include <hip/hip_runtime.h>

#include "fg_act.h"
#include "fg_sched.h"

namespace fg {
namespace gemm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;

// K-tile depth (a multiple of 16).  A compile-time tuning knob: builds may
// override it with -DFG_GEMM_BK=32.
#ifndef FG_GEMM_BK
#define FG_GEMM_BK 16
#endif
constexpr int kBK = FG_GEMM_BK;

// The pipelined whole-tile kernel (gemm_f32_pipe) where the shapes allow; 0
// keeps every call on gemm_f32_mfma.  A compile-time knob for measurement
// builds.
#ifndef FG_GEMM_PIPE
#define FG_GEMM_PIPE 1
#endif
constexpr bool kPipe = FG_GEMM_PIPE != 0;

// Interleaved MFMA blocks for row-contiguous operands in the pipelined
// kernel (gemm_f32_pipe); 0 keeps one block per 32 consecutive rows.  A
// compile-time knob for measurement builds.
#ifndef FG_GEMM_INTERLEAVE
#define FG_GEMM_INTERLEAVE 1
#endif
constexpr bool kInterleave = FG_GEMM_INTERLEAVE != 0;


struct GemmArgs {
    const float *A;
    const float *B;
    float *C;
    float *Z;           // forward: pre-activation output (optional)
    const float *bias;  // forward: row-broadcast bias (optional)
    const float *Zs;    // backward: saved pre-activation for act'(.)
    int M, N, K;
    int lda, ldb, ldc, ldz, ldzs;
    int act;
    int mode;  // 0 forward epilogue, 1 backward (act-derivative) epilogue
    int accumulate;
    int tiles_m, tiles_n;
    int vec_out;  // C (and Z / Zs) rows 16-byte aligned: float4 epilogue I/O
    // TN only: colsum[n] (=|+=) sum_k B[k][n] -- the bias gradient of the
    // layer whose weight gradient this GEMM computes -- taken from the B
    // tiles already in LDS by the workgroups of the first tile row.
    float *colsum;
    int colsum_accumulate;
    // Split K (0: off): workgroup row blockIdx.y multiplies the K slice
    // [ksplit * y, ksplit * (y + 1)) into its own M x N slot of `partial`
    // (row stride N); splitk_reduce then sums the slots in order and applies
    // the epilogue.
    float *partial;
    int ksplit;
    // Prologue (kernels instantiated with PRO != 0): the operand that holds
    // dC -- A of NT (dA = dZ.B^T) or B of TN (dB = A^T.dZ) -- is multiplied
    // elementwise by act'(Pz) as its tiles are loaded, so dZ = dC * act'(Z)
    // is never materialised.  Pz has that operand's shape, row stride ldp.
    const float *Pz;
    int ldp;
};

// Prologue codes (template parameter PRO of the kernels): which operand is
// multiplied by act'(Pz) on load, and which activation.
enum : int { kProNone = 0, kProAReLU = 1, kProAGelu = 2, kProBReLU = 3, kProBGelu = 4 };
constexpr bool pro_on_a(int pro) { return pro == kProAReLU || pro == kProAGelu; }
constexpr bool pro_on_b(int pro) { return pro == kProBReLU || pro == kProBGelu; }
constexpr int pro_act(int pro) {
    return (pro == kProAReLU || pro == kProBReLU) ? kActRelu : kActGelu;
}

// v * act'(z), elementwise (the same fp32 product as the unfused dact pass).
template <int ACT>
__device__ __forceinline__ f32x4 pro_scale(f32x4 v, f32x4 z) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] *= act_grad(ACT, z[e]);
    return v;
}

// The view of split-K workgroup row s: its K slice of A and B, its
// raw-product slot as C, no epilogue.
template <bool AK, bool BNC, int PRO>
__device__ __forceinline__ void split_k_view(GemmArgs &p, int s) {
    if (p.ksplit <= 0) return;
    const int kb = s * p.ksplit;
    p.A += AK ? (size_t)kb : (size_t)kb * p.lda;
    p.B += BNC ? (size_t)kb * p.ldb : (size_t)kb;
    if constexpr (pro_on_a(PRO)) p.Pz += AK ? (size_t)kb : (size_t)kb * p.ldp;
    if constexpr (pro_on_b(PRO)) p.Pz += BNC ? (size_t)kb * p.ldp : (size_t)kb;
    p.K = min(p.ksplit, p.K - kb);
    p.C = p.partial + (size_t)s * p.M * p.N;
    p.ldc = p.N;
    p.mode = 0;
    p.act = kActNone;
    p.bias = nullptr;
    p.Z = nullptr;
    p.accumulate = 0;
    p.colsum = nullptr;
    p.vec_out = p.N % 4 == 0;
}

// Column sums of the B tiles (TN layout, B row-contiguous [k][n]) for the
// workgroups of tile row 0: thread t owns column t % BN and k-rows
// (t / BN) * KPT .. + KPT of each tile; partial sums are combined in a fixed
// order at the end (deterministic).
template <int BN, int BK, int NT>
struct ColSum {
    static constexpr int G = NT >= BN ? NT / BN : 1;  // k-groups
    static constexpr int KPT = BK / G;                // k-rows per thread and tile
    static_assert(NT % BN == 0 && BK % G == 0, "column-sum split");
    float s = 0.0f;
    // Bs(k, c): the tile element at k-row k, column c.
    template <class F>
    __device__ __forceinline__ void add(F Bs) {
        const int c = threadIdx.x % BN, g = threadIdx.x / BN;
#pragma unroll
        for (int i = 0; i < KPT; ++i) s += Bs(g * KPT + i, c);
    }
    // Combines the k-groups through lds (G * BN floats, free) and writes the
    // sums of the tile's columns.  Called by every thread of the workgroup.
    __device__ __forceinline__ void finish(const GemmArgs &p, float *lds, int n0) const {
        const int c = threadIdx.x % BN, g = threadIdx.x / BN;
        lds[g * BN + c] = s;
        __syncthreads();
        if ((int)threadIdx.x < BN && n0 + c < p.N) {
            float t = 0.0f;
#pragma unroll
            for (int k = 0; k < G; ++k) t += lds[k * BN + c];
            float *dst = p.colsum + n0 + c;
            *dst = p.colsum_accumulate ? *dst + t : t;
        }
        __syncthreads();
    }
};

// LDS footprint in floats (NW waves, each staging a 32 x WTN slice in the
// epilogue).
template <int BM, int BN, int BK, bool AK, bool BNC, int WTN, int NW>
struct Lds {
    static constexpr bool a_rowk = AK;    // A stored [row][k] (else [k][row])
    static constexpr bool b_rowk = !BNC;  // B stored [col][k] (else [k][col])
    static constexpr int a_ld = a_rowk ? (BK + 4) : (BM + 4);
    static constexpr int a_sz = a_rowk ? BM * a_ld : BK * a_ld;
    static constexpr int b_ld = b_rowk ? (BK + 4) : (BN + 4);
    static constexpr int b_sz = b_rowk ? BN * b_ld : BK * b_ld;
    static constexpr int buf = a_sz + b_sz;
    static constexpr int stage_ld = WTN + 4;
    static constexpr int stage = NW * 32 * stage_ld;
    static constexpr int total = (2 * buf > stage) ? 2 * buf : stage;
};

// Loads one operand tile into registers with NT threads.  Operand rows are
// M (for A) or N (for B); "KC" = k-contiguous in global memory.
template <int R, int BK, bool KC, bool VEC, int NT>
struct TileLoader {
    static constexpr int kElems = R * BK;
    static constexpr int kPer = VEC ? kElems / 4 / NT : kElems / NT;
    static_assert(kPer >= 1, "tile too small for the thread count");
    static_assert((VEC ? kElems / 4 : kElems) % NT == 0, "tile not divisible");
    f32x4 v4[VEC ? kPer : 1];
    float v1[VEC ? 1 : kPer];

    __device__ __forceinline__ void load(const float *__restrict__ base, int ld, int row0, int rmax,
                                         int k0, int K) {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int idx = threadIdx.x + q * NT;
            if constexpr (VEC) {
                int row, kk;
                if constexpr (KC) {
                    row = idx / (BK / 4);
                    kk = (idx % (BK / 4)) * 4;
                } else {
                    kk = idx / (R / 4);
                    row = (idx % (R / 4)) * 4;
                }
                const int gr = row0 + row, gk = k0 + kk;
                const bool ok = (gr < rmax) && (gk < K);
                const float *p = KC ? base + (size_t)gr * ld + gk : base + (size_t)gk * ld + gr;
                v4[q] = ok ? *reinterpret_cast<const f32x4 *>(p) : f32x4{0.f, 0.f, 0.f, 0.f};
            } else {
                int row, kk;
                if constexpr (KC) {
                    row = idx / BK;
                    kk = idx % BK;
                } else {
                    kk = idx / R;
                    row = idx % R;
                }
                const int gr = row0 + row, gk = k0 + kk;
                const bool ok = (gr < rmax) && (gk < K);
                v1[q] = ok ? (KC ? base[(size_t)gr * ld + gk] : base[(size_t)gk * ld + gr]) : 0.0f;
            }
        }
    }

    // Multiplies the loaded elements by act'(z) of the same elements (z
    // loaded by a loader of the same shape from the prologue tensor).
    template <int ACT>
    __device__ __forceinline__ void scale_by(const TileLoader &z) {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            if constexpr (VEC)
                v4[q] = pro_scale<ACT>(v4[q], z.v4[q]);
            else
                v1[q] *= act_grad(ACT, z.v1[q]);
        }
    }

    __device__ __forceinline__ void store(float *lds) const {
        constexpr int ld = KC ? (BK + 4) : (R + 4);
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int idx = threadIdx.x + q * NT;
            if constexpr (VEC) {
                if constexpr (KC) {
                    const int row = idx / (BK / 4), kk = (idx % (BK / 4)) * 4;
                    *reinterpret_cast<f32x4 *>(lds + row * ld + kk) = v4[q];
                } else {
                    const int kk = idx / (R / 4), row = (idx % (R / 4)) * 4;
                    *reinterpret_cast<f32x4 *>(lds + kk * ld + row) = v4[q];
                }
            } else {
                if constexpr (KC) {
                    const int row = idx / BK, kk = idx % BK;
                    lds[row * ld + kk] = v1[q];
                } else {
                    const int kk = idx / R, row = idx % R;
                    lds[kk * ld + row] = v1[q];
                }
            }
        }
    }
};

// Map the linear workgroup id to an output tile.  Consecutive ids go to
// different XCDs (round-robin dispatch), so first regroup ids per XCD, then
// walk tiles in groups of kGroupM tile-rows, column by column, which keeps
// the A row-panels and B column-panels a group touches small.
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

// One output element of the epilogue.
__device__ __forceinline__ float epi_value(const GemmArgs &p, float v, float bv, int row, int col,
                                           float *zout) {
#pragma clang fp contract(off)
    if (p.mode == 0) {
        v += bv;
        *zout = v;
        return act_fwd(p.act, v);
    }
    if (p.act != kActNone) v *= act_grad(p.act, p.Zs[(size_t)row * p.ldzs + col]);
    return v;
}

// Split K: output (row, col) of the whole product -- the slots' raw
// products summed in slot order, then the epilogue (splitk_reduce and the
// summing blocks of the fused SGD launch, k_optim.hip).
__device__ __forceinline__ void split_sum_store(const GemmArgs &p, int splits, int row, int col) {
    const size_t mn = (size_t)p.M * p.N, i = (size_t)row * p.N + col;
    float v = p.partial[i];
    for (int s = 1; s < splits; ++s) v += p.partial[s * mn + i];
    const float b = (p.mode == 0 && p.bias) ? p.bias[col] : 0.0f;
    float z;
    float o = epi_value(p, v, b, row, col, &z);
    if (p.mode == 0 && p.Z) p.Z[(size_t)row * p.ldz + col] = z;
    float *c = p.C + (size_t)row * p.ldc + col;
    if (p.accumulate) o += *c;  // (in its own statement: no contraction with o)
    *c = o;
}

// Blocks [0, nblocks) of a summing pass over M x N outputs, block b of them
// (kThreads threads, grid-stride).
__device__ __forceinline__ void split_sum_blocks(const GemmArgs &p, int splits, int b,
                                                 int nblocks) {
    const size_t mn = (size_t)p.M * p.N;
    for (size_t i = (size_t)b * kThreads + threadIdx.x; i < mn; i += (size_t)nblocks * kThreads)
        split_sum_store(p, splits, (int)(i / p.N), (int)(i % p.N));
}

// Four consecutive outputs of one row (the vector path of the epilogue):
// the same operations as epi_value per element, with the uniform choices
// (mode, activation, Z, accumulate) taken once per four.  Returns the four
// values stored to C.
__device__ __forceinline__ f32x4 epi_x4(const GemmArgs &p, f32x4 v, f32x4 bv, int row, int col) {
#pragma clang fp contract(off)
    if (p.mode == 0) {
        v += bv;
        if (p.Z) *reinterpret_cast<f32x4 *>(p.Z + (size_t)row * p.ldz + col) = v;
        if (p.act != kActNone) {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = act_fwd(p.act, v[t]);
        }
    } else if (p.act != kActNone) {
        const f32x4 z = *reinterpret_cast<const f32x4 *>(p.Zs + (size_t)row * p.ldzs + col);
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] *= act_grad(p.act, z[t]);
    }
    float *c = p.C + (size_t)row * p.ldc + col;
    if (p.accumulate) v += *reinterpret_cast<const f32x4 *>(c);
    *reinterpret_cast<f32x4 *>(c) = v;
    return v;
}

// Epilogue shared by the GEMM kernels.  Accumulator register r of lane
// (h, l32) in block (i, j) holds C[r0 + 32i + 8(r/4) + 4h + r%4][c0 + 32j + l32]
// (r0, c0: the wave's first row and column); with interleaved blocks (IA =
// TM > 1, IB = TN > 1) row 32i + x becomes TM x + i and column 32j + l32
// becomes TN l32 + j.  Each wave writes one
// 32 x WTN slice to its LDS stage (stride WTN+4 floats), then reads it back
// as float4 rows and applies bias / activation / activation-derivative with
// 16-byte global accesses.  A lane keeps the same four columns through the
// slice (its bias is loaded once) and reads the next row group from LDS
// while it processes the current one.  Each CU runs the epilogue once per
// launch, so its code is fetched cold: the uniform choices sit outside the
// per-element arithmetic and the row loop stays rolled.  lds must hold
// NW * 32 * (WTN + 4) floats and be free (every wave past its last read of
// the operand tiles).
template <int TM, int TN, int WTN, int NW, int IA = 1, int IB = 1>
__device__ __forceinline__ void store_tile(const GemmArgs &p, const f32x16 (&acc)[TM][TN],
                                           float *lds, int r0, int c0, int wave, int lane) {
    static_assert((IA == 1 || IA == TM) && (IB == 1 || IB == TN), "interleave factors");
    constexpr int kStageLd = WTN + 4;
    const int l32 = lane & 31, h = lane >> 5;
    float *stage = lds + wave * (32 * kStageLd);
    constexpr int F4 = WTN / 4;   // float4 per slice row
    constexpr int RPP = 64 / F4;  // slice rows per pass of the wave
    constexpr int NP = 32 / RPP;  // passes per slice
    static_assert(64 % F4 == 0 && 32 % RPP == 0, "epilogue lane mapping");
    const int c4 = (lane % F4) * 4, rr0 = lane / F4;
    const int col = c0 + c4;
    const bool vec = p.vec_out && col + 4 <= p.N;
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (p.mode == 0 && p.bias && vec) bv = *reinterpret_cast<const f32x4 *>(p.bias + col);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                stage[((r >> 2) * 8 + h * 4 + (r & 3)) * kStageLd +
                      (IB > 1 ? TN * l32 + j : j * 32 + l32)] = acc[i][j][r];
        __syncthreads();
        f32x4 nxt = *reinterpret_cast<const f32x4 *>(stage + rr0 * kStageLd + c4);
#pragma unroll 1
        for (int q = 0; q < NP; ++q) {
            const f32x4 v = nxt;
            if (q + 1 < NP)
                nxt = *reinterpret_cast<const f32x4 *>(stage + (rr0 + (q + 1) * RPP) * kStageLd + c4);
            const int row = IA > 1 ? r0 + TM * (rr0 + q * RPP) + i : r0 + i * 32 + rr0 + q * RPP;
            if (row >= p.M || col >= p.N) continue;
            if (vec) {
                (void)epi_x4(p, v, bv, row, col);
            } else {
                float *crow = p.C + (size_t)row * p.ldc;
#pragma unroll 1
                for (int t = 0; t < 4 && col + t < p.N; ++t) {
                    const float b = (p.mode == 0 && p.bias) ? p.bias[col + t] : 0.0f;
                    float z;
                    float o = epi_value(p, v[t], b, row, col + t, &z);
                    if (p.mode == 0 && p.Z) p.Z[(size_t)row * p.ldz + col + t] = z;
                    if (p.accumulate) o += crow[col + t];
                    crow[col + t] = o;
                }
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------ register epilogue
// The pipelined kernels' epilogue when the workgroup's whole tile is in
// bounds and rows are 16-byte aligned: no LDS, no workgroup barrier.
// Accumulator registers 4k .. 4k+3 of lane (h, l32) hold rows x = 8k + 4h +
// 0..3 of a block's column; the block's rows and columns in C follow
// store_tile's mapping (interleaved or not).  Without column interleave, a
// 4x4 transpose within each quad of lanes (quad_transpose4) leaves lane e of
// quad a with row x = 8k + 4h + e and columns 4a .. 4a+3, finished and
// stored as 16 bytes; with it (IB = TN, the TN layout's weight gradients) a
// lane already holds TN consecutive columns of each row and stores them as
// they are, for the plain product only (the kinds with a bias, an
// activation or Z take store_tile there).  The kind of epilogue is a
// template parameter, so the per-element code branches on none of it; the
// operations per element are epi_x4's (a plain product still adds the zero
// bias, as epi_x4 does, which turns -0 into +0), so the bits are
// store_tile's.  Four row groups k of a block run as a loop that picks its
// registers by k, which keeps the code (fetched cold, once per CU and
// launch) short.  The staged epilogue cost 5-23 us per launch on the c5
// shapes (its LDS round trip, barriers and a pass loop branching on every
// epilogue choice; the activation-derivative kinds also waited for each
// saved pre-activation load in turn).
template <int MODE, int ACT>
__device__ __forceinline__ void epi_x4_k(const GemmArgs &p, f32x4 v, f32x4 bv, f32x4 z, int row,
                                         int col) {
#pragma clang fp contract(off)
    if constexpr (MODE == 0) {
        v += bv;
        if (p.Z) *reinterpret_cast<f32x4 *>(p.Z + (size_t)row * p.ldz + col) = v;
        if constexpr (ACT != kActNone) {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = act_fwd(ACT, v[t]);
        }
    } else if constexpr (ACT != kActNone) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] *= act_grad(ACT, z[t]);
    }
    float *c = p.C + (size_t)row * p.ldc + col;
    if (p.accumulate) v += *reinterpret_cast<const f32x4 *>(c);
    *reinterpret_cast<f32x4 *>(c) = v;
}

template <int TM, int TN, int IA, int IB, int MODE, int ACT>
__device__ __forceinline__ void store_direct_k(const GemmArgs &p, const f32x16 (&acc)[TM][TN],
                                               int r0, int c0, int lane) {
#pragma clang fp contract(off)
    const int l32 = lane & 31, h = lane >> 5, e = lane & 3;
    // Row of C of block row i and block-row index x (0..31).
    auto crow = [&](int i, int x) { return IA > 1 ? r0 + TM * x + i : r0 + 32 * i + x; };
    if constexpr (IB == 1) {
        const int a4 = l32 & ~3;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = c0 + 32 * j + a4;
            f32x4 bv = {0.f, 0.f, 0.f, 0.f};
            if (MODE == 0 && p.bias) bv = *reinterpret_cast<const f32x4 *>(p.bias + col);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const f32x16 &a = acc[i][j];
                constexpr bool kZs = MODE == 1 && ACT != kActNone;
                f32x4 zr[4];
                if constexpr (kZs) {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        zr[k] = *reinterpret_cast<const f32x4 *>(
                            p.Zs + (size_t)crow(i, 8 * k + 4 * h + e) * p.ldzs + col);
                }
#pragma unroll 1
                for (int k = 0; k < 4; ++k) {
                    f32x4 x;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        x[q] = k == 0 ? a[q] : k == 1 ? a[4 + q] : k == 2 ? a[8 + q] : a[12 + q];
                    const f32x4 y = quad_transpose4(x, e);
                    f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    if constexpr (kZs) z = k == 0 ? zr[0] : k == 1 ? zr[1] : k == 2 ? zr[2] : zr[3];
                    epi_x4_k<MODE, ACT>(p, y, bv, z, crow(i, 8 * k + 4 * h + e), col);
                }
            }
        }
    } else {
        typedef float vec_t __attribute__((ext_vector_type(IB)));
        const int col = c0 + TN * l32;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll 1
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    vec_t v;
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const f32x16 &a = acc[i][j];
                        v[j] = (k == 0 ? a[q] : k == 1 ? a[4 + q] : k == 2 ? a[8 + q] : a[12 + q]) +
                               0.0f;
                    }
                    float *c = p.C + (size_t)crow(i, 8 * k + 4 * h + q) * p.ldc + col;
                    if (p.accumulate) v += *reinterpret_cast<const vec_t *>(c);
                    *reinterpret_cast<vec_t *>(c) = v;
                }
    }
}

// Runs the register epilogue's kind for p; false (nothing stored) for a
// kind it does not take, which then goes to store_tile.  An activation code
// outside ReLU / GELU takes the kind without one (act_fwd / act_grad are
// the identity for it, so the bits agree).  Waves holding 256 accumulator
// registers (the 4-wave 256x256 tile) keep store_tile: with every register
// taken, the register epilogue's temporaries spill.
template <int TM, int TN, int IA, int IB>
__device__ __forceinline__ bool store_direct(const GemmArgs &p, const f32x16 (&acc)[TM][TN],
                                             int r0, int c0, int lane) {
    if constexpr (TM * TN > 8) {
        return false;
    } else if constexpr (IB > 1) {
        if (p.mode != 0 || p.bias || p.Z || p.act == kActRelu || p.act == kActGelu) return false;
        store_direct_k<TM, TN, IA, IB, 0, kActNone>(p, acc, r0, c0, lane);
    } else if (p.mode == 0) {
        if (p.act == kActRelu) store_direct_k<TM, TN, IA, IB, 0, kActRelu>(p, acc, r0, c0, lane);
        else if (p.act == kActGelu) store_direct_k<TM, TN, IA, IB, 0, kActGelu>(p, acc, r0, c0, lane);
        else store_direct_k<TM, TN, IA, IB, 0, kActNone>(p, acc, r0, c0, lane);
    } else {
        if (p.act == kActRelu) store_direct_k<TM, TN, IA, IB, 1, kActRelu>(p, acc, r0, c0, lane);
        else if (p.act == kActGelu) store_direct_k<TM, TN, IA, IB, 1, kActGelu>(p, acc, r0, c0, lane);
        else store_direct_k<TM, TN, IA, IB, 1, kActNone>(p, acc, r0, c0, lane);
    }
    return true;
}

// The kernel bodies take their workgroup's coordinates (bx: output tile,
// by: K slice) as arguments, so that a launch of two independent GEMMs
// (gemm_pair, k_gemm_pair.hip) can run either body in a workgroup.
template <int BM, int BN, int BK, int WGM, int WGN, bool AK, bool BNC, bool VEC, int PRO>
__device__ __forceinline__ void gemm_f32_mfma_body(GemmArgs p, int bx, int by) {
    split_k_view<AK, BNC, PRO>(p, by);
    constexpr int NT = 64 * WGM * WGN;
    static_assert(WGM * WGN == 4 || WGM * WGN == 8, "4 or 8 waves per workgroup");
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
    static_assert(BK % 16 == 0, "BK must be a multiple of 16");
    using L = Lds<BM, BN, BK, AK, BNC, WTN, WGM * WGN>;
    __shared__ __attribute__((aligned(16))) float lds[L::total];

    int tile_m, tile_n;
    tile_of(bx, p.tiles_m, p.tiles_n, tile_m, tile_n);
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

    TileLoader<BM, BK, AK, VEC, NT> la;
    TileLoader<BN, BK, !BNC, VEC, NT> lb;
    // Prologue: act' tiles of the operand that holds dC (loaded with it).
    TileLoader<BM, BK, AK, VEC, NT> za;
    TileLoader<BN, BK, !BNC, VEC, NT> zb;
    const int nk = (p.K + BK - 1) / BK;
    constexpr bool kTN = !AK && BNC;
    ColSum<BN, BK, NT> cs;
    const bool do_cs = kTN && p.colsum && tile_m == 0;
    auto load_tiles = [&](int k0) {
        la.load(p.A, p.lda, m0, p.M, k0, p.K);
        lb.load(p.B, p.ldb, n0, p.N, k0, p.K);
        if constexpr (pro_on_a(PRO)) za.load(p.Pz, p.ldp, m0, p.M, k0, p.K);
        if constexpr (pro_on_b(PRO)) zb.load(p.Pz, p.ldp, n0, p.N, k0, p.K);
    };
    auto store_tiles = [&](float *dst) {
        if constexpr (pro_on_a(PRO)) la.template scale_by<pro_act(PRO)>(za);
        if constexpr (pro_on_b(PRO)) lb.template scale_by<pro_act(PRO)>(zb);
        la.store(dst);
        lb.store(dst + L::a_sz);
    };

    load_tiles(0);
    store_tiles(lds);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) load_tiles((kt + 1) * BK);
        const float *As = lds + cur * L::buf;
        const float *Bs = As + L::a_sz;
        // Group g of the tile (4 consecutive k per lane half): lane half h
        // feeds k = 16*(g/2) + 8h + 4*(g%2) + s to the s-th MFMA.
        auto load_frag = [&](int g, f32x4 *a, f32x4 *b) {
            const int kb = (g >> 1) * 16 + 8 * h + 4 * (g & 1);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int row = wm0 + i * 32 + l32;
                if constexpr (L::a_rowk) {
                    a[i] = *reinterpret_cast<const f32x4 *>(As + row * L::a_ld + kb);
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s) a[i][s] = As[(kb + s) * L::a_ld + row];
                }
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = wn0 + j * 32 + l32;
                if constexpr (!L::b_rowk) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) b[j][s] = Bs[(kb + s) * L::b_ld + col];
                } else {
                    b[j] = *reinterpret_cast<const f32x4 *>(Bs + col * L::b_ld + kb);
                }
            }
        };
        auto mfma_group = [&](const f32x4 *a, const f32x4 *b) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s],
                                                                         acc[i][j], 0, 0, 0);
        };
        constexpr int NG = BK / 8;  // 4-k groups per tile and lane half
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            f32x4 a[TM], b[TN];
            load_frag(g, a, b);
            mfma_group(a, b);
        }
        if constexpr (kTN)
            if (do_cs) cs.add([&](int k, int c) { return Bs[k * L::b_ld + c]; });
        if (more) store_tiles(lds + (cur ^ 1) * L::buf);
        __syncthreads();
    }

    if constexpr (kTN)
        if (do_cs) cs.finish(p, lds, n0);
    store_tile<TM, TN, WTN, WGM * WGN>(p, acc, lds, m0 + wm0, n0 + wn0, wave, lane);
}

// ------------------------------------------------ pipelined variant
// The same GEMM, software-pipelined over whole K tiles: used when every
// 16-byte chunk of a tile is either in bounds or belongs only to outputs that
// are masked (K % BK == 0 and the VEC alignment conditions).  Rows (or
// columns) past the matrix edge are clamped to the last valid one, so every
// load reads mapped memory; the values they bring only reach masked outputs.
// Each wave loads its share of a tile as 16 bytes per lane; lane l's chunk of
// wave load li lands at LDS float offset li * 256 + 4 l of the operand's
// stage area, and the source address of that chunk is chosen so that the
// stage ends up in the swizzled layout below.  Two ways to move the chunks:
//  * staged (every tile but 256x256): global loads into registers, two
//    register sets alternating by tile parity, written to a two-stage LDS
//    ring by ds_write_b128 one tile later;
//  * direct (256x256, whose accumulators leave no room for two register
//    sets): global_load_lds_dwordx4 straight into a three-stage LDS ring
//    (two stages where three do not fit).
// Measured on gfx950 (2048x4096x4096 NN, same inputs): MFMA busy 87.5 % with
// direct loads for every tile, 90.4 % with staged loads; direct loads cost
// the same whether they come from HBM or from L2, so it is the asynchronous
// LDS writes, not memory, that the staged path saves.
//
// LDS layout per stage (no padding -- each wave load fills a whole 1 KiB run):
//  * a k-contiguous operand [rows][BK], 16-byte chunk c of row r stored at
//    chunk c ^ ((r / (64 / BK)) % (BK / 4)): the 8 rows read together by a
//    16-byte LDS read then hit distinct banks;
//  * a row-contiguous operand [BK][R] (R = BM or BN), chunk c of k-row k
//    stored at chunk c ^ (8 * ((k / 8) % 2)): the two lane halves, which read
//    k-rows 8 apart, hit opposite halves of the banks.
template <int BK>
__device__ __forceinline__ int swz_k(int row) {
    return (row / (64 / BK)) % (BK / 4);
}
__device__ __forceinline__ int swz_r(int k) { return ((k >> 3) & 1) * 8; }

template <int BM, int BN, int BK, int WGM, int WGN, bool AK, bool BNC, bool VEC, int PRO>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_f32_mfma(GemmArgs p) {
    gemm_f32_mfma_body<BM, BN, BK, WGM, WGN, AK, BNC, VEC, PRO>(p, blockIdx.x, blockIdx.y);
}

// KT: K need not be a multiple of BK (staged tiles, no prologue): the tile
// loop runs over the whole tiles only, and the K % BK values of k past them
// are multiplied into the accumulators straight from global memory at the
// end (see the K tail below), so the loop keeps the whole-tile addressing.
// LDS of the pipelined kernel, in floats: its stages (staged tiles: two;
// direct: three when they fit in the 160 KiB of LDS, else two) or the
// epilogue's staging, whichever is larger.
template <int BM, int BN, int BK, int WGM, int WGN>
struct PipeLds {
    static constexpr int kStageSz = BM * BK + BN * BK;
    static constexpr bool kStaged = !(BM == 256 && BN == 256);
    static constexpr int kStages = kStaged ? 2 : 3 * kStageSz * 4 <= 160 * 1024 ? 3 : 2;
    static constexpr int kEpi = WGM * WGN * 32 * (BN / WGN + 4);
    static constexpr int floats = (kStages * kStageSz > kEpi) ? kStages * kStageSz : kEpi;
};

// The kernel's LDS buffer of N floats: one static array per N, so bodies
// that ask for the same N in one launch share it.
template <int N>
__device__ __forceinline__ float (&lds_buffer())[N] {
    __shared__ __attribute__((aligned(16))) float buf[N];
    return buf;
}

// LDSN: the LDS buffer's size in floats, at least PipeLds::floats (0: just
// that) -- a launch running several bodies gives them all the largest one.
template <int BM, int BN, int BK, int WGM, int WGN, bool AK, bool BNC, int PRO, bool KT,
          int LDSN = 0>
__device__ __forceinline__ void gemm_f32_pipe_body(GemmArgs p, int bx, int by) {
    split_k_view<AK, BNC, PRO>(p, by);
    constexpr int NW = WGM * WGN;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
    static_assert(BK == 16 || BK == 32, "BK 16 or 32");
    constexpr int kInstA = BM * BK / 4 / 64, kInstB = BN * BK / 4 / 64;  // wave loads per tile
    static_assert(kInstA % NW == 0 && kInstB % NW == 0, "loads divide among the waves");
    constexpr int kPerA = kInstA / NW, kPerB = kInstB / NW, kLoads = kPerA + kPerB;
    using PL = PipeLds<BM, BN, BK, WGM, WGN>;
    constexpr int kASz = BM * BK, kStageSz = PL::kStageSz;
    constexpr bool kStaged = PL::kStaged;
    // The prologue scales a tile in registers, between its load and its LDS
    // write: staged tiles only.
    static_assert(PRO == kProNone || kStaged, "prologue needs the staged path");
    static_assert(!KT || (kStaged && PRO == kProNone), "K tail: staged tiles, no prologue");
    constexpr int kStages = PL::kStages;
    static_assert(LDSN == 0 || LDSN >= PL::floats, "LDS buffer too small");
    float(&lds)[LDSN ? LDSN : PL::floats] = lds_buffer<LDSN ? LDSN : PL::floats>();

    int tile_m, tile_n;
    tile_of(bx, p.tiles_m, p.tiles_n, tile_m, tile_n);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    // The wave index as a uniform (scalar) value: it selects each wave's LDS
    // destinations, which the compiler would otherwise treat as varying.
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

    // Source address of this lane's chunk for wave load `li` of an operand:
    // the chunk's position in the stage fixes (row, physical chunk); the
    // swizzle gives the logical chunk to fetch.
    auto src_kc = [&](const float *base, int ld, int r0, int rmax, int k0, int pos) {
        const int row = pos / (BK / 4), pc = pos % (BK / 4);
        const int c = pc ^ swz_k<BK>(row);
        const float *rp = base + (size_t)min(r0 + row, rmax - 1) * ld;
        // Whole tiles: the per-lane part (row, chunk) stays loop-invariant
        // and k0 is added as a uniform offset.
        return rp + 4 * c + k0;
    };
    auto src_rc = [&](const float *base, int ld, int r0, int rmax, int k0, int pos, int R) {
        const int k = pos / (R / 4), pc = pos % (R / 4);
        const int c = pc ^ swz_r(k);
        return base + (size_t)(k0 + k) * ld + min(r0 + 4 * c, rmax - 4);
    };
    // Wave load q (0 .. kLoads-1) of a tile: this wave's share of A first,
    // then of B.  Source of this lane's chunk, and its place in a stage.
    auto src_of = [&](int kt, int q) -> const float * {
        const int k0 = kt * BK;
        if (q < kPerA) {
            const int pos = (wave * kPerA + q) * 64 + lane;
            return AK ? src_kc(p.A, p.lda, m0, p.M, k0, pos)
                      : src_rc(p.A, p.lda, m0, p.M, k0, pos, BM);
        }
        const int pos = (wave * kPerB + (q - kPerA)) * 64 + lane;
        return BNC ? src_rc(p.B, p.ldb, n0, p.N, k0, pos, BN) : src_kc(p.B, p.ldb, n0, p.N, k0, pos);
    };
    auto run_of = [&](int stage, int q) -> float * {  // the wave load's 1 KiB run
        float *sa = lds + stage * kStageSz;
        return q < kPerA ? sa + (wave * kPerA + q) * 256 : sa + kASz + (wave * kPerB + q - kPerA) * 256;
    };
    // (Source and destination are formed here rather than taken from src_of
    // / run_of: the LDS-load builtin fed from those lambdas' return values
    // makes the host compilation pass drop the kernel's launch stub without a
    // diagnostic.)
    auto issue_direct = [&](int kt, int stage, int q) {
        float *sa = lds + stage * kStageSz;
        const int k0 = kt * BK;
        if (q < kPerA) {
            const int li = wave * kPerA + q, pos = li * 64 + lane;
            const float *src = AK ? src_kc(p.A, p.lda, m0, p.M, k0, pos)
                                  : src_rc(p.A, p.lda, m0, p.M, k0, pos, BM);
            __builtin_amdgcn_global_load_lds(src, sa + li * 256, 16, 0, 0);
        } else {
            const int li = wave * kPerB + (q - kPerA), pos = li * 64 + lane;
            const float *src = BNC ? src_rc(p.B, p.ldb, n0, p.N, k0, pos, BN)
                                   : src_kc(p.B, p.ldb, n0, p.N, k0, pos);
            __builtin_amdgcn_global_load_lds(src, sa + kASz + li * 256, 16, 0, 0);
        }
    };
    auto load_reg = [&](int kt, int q) { return *reinterpret_cast<const f32x4 *>(src_of(kt, q)); };
    auto store_reg = [&](int stage, int q, const f32x4 &v) {
        *reinterpret_cast<f32x4 *>(run_of(stage, q) + 4 * lane) = v;
    };
    // Prologue: each wave load of the operand that holds dC (loads
    // kProFirst .. kProFirst+kPro-1) is paired with a load of Pz at the same
    // position; the chunk is multiplied by act'(Pz) before its LDS write.
    constexpr int kPro = pro_on_a(PRO) ? kPerA : pro_on_b(PRO) ? kPerB : 0;
    constexpr int kProFirst = pro_on_a(PRO) ? 0 : kPerA;
    constexpr int kProN = kPro > 0 ? kPro : 1;  // register-set size
    auto is_pro = [](int q) { return q >= kProFirst && q < kProFirst + kPro; };
    auto load_pz = [&](int kt, int q) -> f32x4 {
        const int k0 = kt * BK;
        const float *src;
        if constexpr (pro_on_a(PRO)) {
            const int pos = (wave * kPerA + q) * 64 + lane;
            src = AK ? src_kc(p.Pz, p.ldp, m0, p.M, k0, pos)
                     : src_rc(p.Pz, p.ldp, m0, p.M, k0, pos, BM);
        } else {
            const int pos = (wave * kPerB + (q - kPerA)) * 64 + lane;
            src = BNC ? src_rc(p.Pz, p.ldp, n0, p.N, k0, pos, BN)
                      : src_kc(p.Pz, p.ldp, n0, p.N, k0, pos);
        }
        return *reinterpret_cast<const f32x4 *>(src);
    };
    // Chunk q of register set (R, Z) as it goes to LDS.
    auto staged_value = [&](const f32x4 *R, const f32x4 *Zr, int q, int) -> f32x4 {
        if constexpr (PRO != kProNone)
            if (is_pro(q)) return pro_scale<pro_act(PRO)>(R[q], Zr[q - kProFirst]);
        return R[q];
    };

    const int nk = p.K / BK;  // whole tiles (KT: the rest is the K tail)
    constexpr bool kTN = !AK && BNC;
    ColSum<BN, BK, 64 * NW> cs;
    const bool do_cs = kTN && p.colsum && tile_m == 0;

    // Fragments of 4-k group g (of BK / 8) of a stage: lane half h holds k
    // 8h .. 8h+3 of the group's 16-k block, so the 4 MFMA steps of the
    // group cover all 16 k across both halves.
    auto k_of = [&](int g) { return (g >> 1) * 16 + 8 * h + 4 * (g & 1); };
    auto frag_a = [&](const float *As, int g, int i) {
        const int kb = k_of(g), row = wm0 + i * 32 + l32;
        f32x4 a;
        if constexpr (AK) {
            const int c = (kb >> 2) ^ swz_k<BK>(row);
            a = *reinterpret_cast<const f32x4 *>(As + row * BK + 4 * c);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int k = kb + s;
                a[s] = As[k * BM + ((((row >> 2) ^ swz_r(k)) << 2) | (row & 3))];
            }
        }
        return a;
    };
    auto frag_b = [&](const float *Bs, int g, int j) {
        const int kb = k_of(g), col = wn0 + j * 32 + l32;
        f32x4 b;
        if constexpr (BNC) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int k = kb + s;
                b[s] = Bs[k * BN + ((((col >> 2) ^ swz_r(k)) << 2) | (col & 3))];
            }
        } else {
            const int c = (kb >> 2) ^ swz_k<BK>(col);
            b = *reinterpret_cast<const f32x4 *>(Bs + col * BK + 4 * c);
        }
        return b;
    };
    // Row-contiguous operands with more than one MFMA block per wave are
    // interleaved: block i of A covers wave rows TM r + i (r = 0..31) and
    // block j of B wave columns TN c + j, so a lane's operands for all its
    // blocks at one k are TM (TN) consecutive floats -- one ds_read_b64 /
    // b128 per k step instead of TM (TN) scalar reads.  The fragment
    // registers then hold, at flat position s T + block, the value of k step
    // s; store_tile maps the blocks back.
    // Used in the TN layout (both operands row-contiguous: +1.7 % on the
    // 256-row tiles); for NN's B operand the four extra read units crowd
    // the MFMA slots that also carry the staged tile loads (-6 % on the
    // 256x128 8-wave tile), so NN keeps one block per 32 columns.
    constexpr bool kIl = kInterleave && !AK && BNC;
    constexpr int IA = (kIl && TM > 1) ? TM : 1;
    constexpr int IB = (kIl && TN > 1) ? TN : 1;
    static_assert(IA == 1 || IA == 2 || IA == 4, "A interleave of 2 or 4 blocks");
    static_assert(IB == 1 || IB == 2 || IB == 4, "B interleave of 2 or 4 blocks");
    constexpr int NRA = IA > 1 ? 4 : TM;  // LDS read units of A per group
    constexpr int NRB = IB > 1 ? 4 : TN;
    static_assert(NRA + NRB <= 4 * TM * TN, "one read unit per MFMA slot");
    // T consecutive floats at `src` into flat positions s T .. s T + T - 1.
    auto read_run = [&](const float *src, int s, auto &f) {
        constexpr int T = sizeof(f) / sizeof(f32x4);
        if constexpr (T == 4) {
            f[s] = *reinterpret_cast<const f32x4 *>(src);
        } else {
            typedef float f32x2 __attribute__((ext_vector_type(2)));
            const f32x2 v = *reinterpret_cast<const f32x2 *>(src);
            f[s >> 1][2 * (s & 1)] = v[0];
            f[s >> 1][2 * (s & 1) + 1] = v[1];
        }
    };
    // Read unit u of group g: block u (k-contiguous, or one block per wave),
    // or k step u of every block (interleaved).
    auto read_a = [&](const float *As, int g, int u, f32x4 (&a)[TM]) {
        if constexpr (IA > 1) {
            const int k = k_of(g) + u, row = wm0 + TM * l32;
            read_run(As + k * BM + ((((row >> 2) ^ swz_r(k)) << 2) | (row & 3)), u, a);
        } else {
            a[u] = frag_a(As, g, u);
        }
    };
    auto read_b = [&](const float *Bs, int g, int u, f32x4 (&b)[TN]) {
        if constexpr (IB > 1) {
            const int k = k_of(g) + u, col = wn0 + TN * l32;
            read_run(Bs + k * BN + ((((col >> 2) ^ swz_r(k)) << 2) | (col & 3)), u, b);
        } else {
            b[u] = frag_b(Bs, g, u);
        }
    };
    auto frag = [&](const float *As, const float *Bs, int g, f32x4 (&a)[TM], f32x4 (&b)[TN]) {
#pragma unroll
        for (int u = 0; u < NRA; ++u) read_a(As, g, u, a);
#pragma unroll
        for (int u = 0; u < NRB; ++u) read_b(Bs, g, u, b);
    };
    // MFMA m (of 4 TM TN) of a group: k step m / (TM TN), then i, then j,
    // so consecutive MFMAs update different accumulators.
    auto mfma_one = [&](const f32x4 (&a)[TM], const f32x4 (&b)[TN], int m) {
        const int s = m / (TM * TN), i = (m / TN) % TM, j = m % TN;
        const int fa = IA > 1 ? s * TM + i : i * 4 + s, fb = IB > 1 ? s * TN + j : j * 4 + s;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[fa >> 2][fa & 3], b[fb >> 2][fb & 3],
                                                         acc[i][j], 0, 0, 0);
    };    auto colsum_add = [&](const float *Bs) {
        if constexpr (kTN)
            if (do_cs)
                cs.add([&](int k, int c) {
                    return Bs[k * BN + ((((c >> 2) ^ swz_r(k)) << 2) | (c & 3))];
                });
    };
    constexpr int NG = BK / 8;

    // Barrier-overlapped loop: the last 8-k group of tile kt is read into
    // registers before the barrier that ends tile kt and multiplied after
    // it, so the matrix units stay busy across the barrier while the first
    // operands of tile kt+1 are read.  Tile t lives in stage t % kStages.
    // The prologue issues tiles 0 .. kAhead-1; iteration kt issues tile
    // kt + kAhead into the stage of tile kt-1, which every wave finished
    // reading before the barrier that ended tile kt-1.  Past the last tile
    // an iteration reloads tile nk-1 into that free stage, which nothing
    // reads again: the loop body has no branch, so its loads are scheduled
    // among the MFMAs of its first group, and every iteration leaves the
    // same kAhead tiles in flight.
    // Each group runs its MFMAs in a fixed order: after MFMA m, the reads of
    // read unit m of the next group (A units, then B) and, in the first
    // group of a tile, the tile's memory operations (`mem(m)`).  Reads or
    // loads issued in a burst fill the wave's memory queues and hold up the
    // MFMAs behind them, which no other wave hides when a SIMD runs one
    // (measured: issuing the reads first, or the loads on consecutive MFMAs,
    // costs up to 10 % on the 4-wave tiles).
    constexpr int kMfma = 4 * TM * TN;
    static_assert(kLoads >= 1 && kLoads <= kMfma, "at most one load per MFMA");
    constexpr int kAhead = kStages - 1;     // direct: tiles in flight
    constexpr int kStride = kMfma / kLoads;  // direct: MFMAs per load
    // One group's MFMAs on (ca, cb).  With `ld` (the first group of a tile)
    // the tile's memory operations go out among them: staged, after MFMA m <
    // kLoads, register set Rw's chunk m is written to stage `slot` and its
    // register refilled from tile kl (Rl); direct, every kStride-th MFMA
    // issues one load of tile kl into stage `slot`.
    auto run_group = [&](const f32x4 (&ca)[TM], const f32x4 (&cb)[TN], const float *An,
                         const float *Bn, int gn, f32x4 (&na)[TM], f32x4 (&nb)[TN], bool ld,
                         int kl, int slot, const f32x4 *Rw, f32x4 *Rl, const f32x4 *Zw,
                         f32x4 *Zl, int kst) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < kMfma; ++m) {
            mfma_one(ca, cb, m);
            if (m < NRA)
                read_a(An, gn, m, na);
            else if (m < NRA + NRB)
                read_b(Bn, gn, m - NRA, nb);
            if (ld) {
                if constexpr (kStaged) {
                    if (m < kLoads) {
                        store_reg(slot, m, staged_value(Rw, Zw, m, kst));
                        Rl[m] = load_reg(kl, m);
                        if constexpr (PRO != kProNone)
                            if (is_pro(m)) Zl[m - kProFirst] = load_pz(kl, m);
                    }
                } else {
                    if (m % kStride == 0 && m / kStride < kLoads) issue_direct(kl, slot, m / kStride);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Operands double-buffered in registers: the LDS reads of group g+1 are
    // issued among the MFMAs of group g, so the matrix units never wait for
    // the reads of the group they are about to run; ca / cb hold the
    // operands of the next group to multiply.  The loop is barrier-
    // overlapped: the last group of tile kt is read into registers before
    // the barrier that ends tile kt and multiplied after it, while the first
    // operands of tile kt+1 are read, so the matrix units stay busy across
    // the barrier.  Past that barrier every wave holds all of tile kt's
    // operands and its stage may be refilled.
    f32x4 ca[TM], cb[TN];
    auto tile = [&](int kt, int kl, int slot, const f32x4 *Rw, f32x4 *Rl, const f32x4 *Zw,
                    f32x4 *Zl) {
        const float *As = lds + (kt % kStages) * kStageSz;
        const float *Bs = As + kASz;
        const int kst = min(kt + 1, nk - 1);  // staged: the tile Rw holds
#pragma unroll
        for (int g = 0; g < NG - 1; ++g) {
            // Group g's operands (read during the previous group) have
            // landed; waiting here, before the next group's reads are
            // issued, leaves those in flight behind the MFMAs.
            wait_lgkm0();
            f32x4 na[TM], nb[TN];
            run_group(ca, cb, As, Bs, g + 1, na, nb, g == 0, kl, slot, Rw, Rl, Zw, Zl, kst);
#pragma unroll
            for (int i = 0; i < TM; ++i) ca[i] = na[i];
#pragma unroll
            for (int j = 0; j < TN; ++j) cb[j] = nb[j];
        }
        colsum_add(Bs);
        // ca / cb: the last group of tile kt.  Every wave's reads (and LDS
        // writes) of this tile are done before the barrier; direct, this
        // wave's loads of tile kt+1 are done once at most the newest
        // kAhead-1 tiles' are outstanding, and the barrier publishes every
        // wave's.
        wait_lgkm0();
        if constexpr (!kStaged) wait_vmcnt<(kAhead - 1) * kLoads>();
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_barrier" ::: "memory");
        // Group 0 of tile kt+1 (past the last tile: a stage nothing uses,
        // read and discarded).
        f32x4 na[TM], nb[TN];
        const float *An = lds + ((kt + 1) % kStages) * kStageSz;
        run_group(ca, cb, An, An + kASz, 0, na, nb, false, 0, 0, Rw, Rl, Zw, Zl, 0);
#pragma unroll
        for (int i = 0; i < TM; ++i) ca[i] = na[i];
#pragma unroll
        for (int j = 0; j < TN; ++j) cb[j] = nb[j];
    };
    if constexpr (kStaged) {
        // Tile t is loaded into register set t % 2 during tile t-2 (one load
        // after each of the first kLoads MFMAs of the tile's first group),
        // and written from there to stage t % 2 during tile t-1 (the stage of
        // tile t-2, free since the barrier that ended tile t-2); each write
        // goes out right before the load that refills its registers.  Past
        // the last tile, tile nk-1 is reloaded and written to the free stage,
        // which nothing reads.  The kt loop is unrolled by two so that the
        // register sets swap roles without copies.
        if (nk > 0) {
            f32x4 R0[kLoads], R1[kLoads];
            f32x4 Z0[kProN], Z1[kProN];  // prologue chunks (unused without PRO)
#pragma unroll
            for (int q = 0; q < kLoads; ++q) {
                R0[q] = load_reg(0, q);
                if constexpr (PRO != kProNone)
                    if (is_pro(q)) Z0[q - kProFirst] = load_pz(0, q);
            }
#pragma unroll
            for (int q = 0; q < kLoads; ++q) {
                R1[q] = load_reg(min(1, nk - 1), q);
                if constexpr (PRO != kProNone)
                    if (is_pro(q)) Z1[q - kProFirst] = load_pz(min(1, nk - 1), q);
            }
#pragma unroll
            for (int q = 0; q < kLoads; ++q) store_reg(0, q, staged_value(R0, Z0, q, 0));
            wait_lgkm0();
            asm volatile("s_barrier" ::: "memory");
            frag(lds, lds + kASz, 0, ca, cb);
            // Tile kt writes the set holding tile kt+1 and refills the other
            // with tile kt+2; that set was loaded a whole tile ago.
            int kt = 0;
            for (; kt + 1 < nk; kt += 2) {
                wait_vmcnt<0>();
                tile(kt, min(kt + 2, nk - 1), (kt + 1) % kStages, R1, R0, Z1, Z0);
                wait_vmcnt<0>();
                tile(kt + 1, min(kt + 3, nk - 1), kt % kStages, R0, R1, Z0, Z1);
            }
            if (kt < nk) {
                wait_vmcnt<0>();
                tile(kt, nk - 1, (kt + 1) % kStages, R1, R0, Z1, Z0);
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
            for (int t = 0; t < kAhead; ++t)
#pragma unroll
                for (int q = 0; q < kLoads; ++q) issue_direct(min(t, nk - 1), t, q);
            wait_vmcnt<(kAhead - 1) * kLoads>();  // tile 0 landed
            asm volatile("s_barrier" ::: "memory");
            frag(lds, lds + kASz, 0, ca, cb);
            for (int kt = 0; kt < nk; ++kt)
                tile(kt, min(kt + kAhead, nk - 1), (kt + kAhead) % kStages, nullptr, nullptr,
                     nullptr, nullptr);
            wait_vmcnt<0>();  // the reloads past the last tile, before the LDS reuse
        }
    }
    // K tail (KT): k = kb .. K-1 past the whole tiles, multiplied straight
    // from global memory in the order the tile loop takes a tile (MFMA step
    // s of group g, blocks i then j; lane half h supplies k = kb + k_of(g) +
    // s), as from a last tile zero-filled past K: a group whose k are all
    // past K is skipped, and a lane supplies zeros for its k past K.  A lane
    // takes the four k of a group from a k-contiguous operand with one
    // 16-byte load (K % 4 == 0 there), from a row-contiguous one with four
    // loads that are coalesced across the lanes; every address is clamped
    // into the operand, and all loads go out before the first MFMA.  The
    // column sums (TN) take the same k, after the tiles'.
    if constexpr (KT) {
        const int kb = nk * BK;
        if (kb < p.K) {
            int arow[TM], bcol[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                arow[i] = min(m0 + wm0 + (IA > 1 ? TM * l32 + i : 32 * i + l32), p.M - 1);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bcol[j] = min(n0 + wn0 + (IB > 1 ? TN * l32 + j : 32 * j + l32), p.N - 1);
            // Four k from k4 of row r of a k-contiguous operand, or of
            // column r of a row-contiguous one; zeros past K.
            auto four = [&](const float *base, int ld, bool kc, int r, int k4) {
                f32x4 v;
                if (kc) {
                    v = *reinterpret_cast<const f32x4 *>(base + (size_t)r * ld + min(k4, p.K - 4));
                    if (k4 >= p.K) v = f32x4{0.f, 0.f, 0.f, 0.f};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x = base[(size_t)min(k4 + e, p.K - 1) * ld + r];
                        v[e] = k4 + e < p.K ? x : 0.0f;
                    }
                }
                return v;
            };
            f32x4 ta[NG][TM], tb[NG][TN];
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                if (kb + (g >> 1) * 16 + 4 * (g & 1) >= p.K) continue;  // uniform
                const int k4 = kb + k_of(g);
#pragma unroll
                for (int i = 0; i < TM; ++i) ta[g][i] = four(p.A, p.lda, AK, arow[i], k4);
#pragma unroll
                for (int j = 0; j < TN; ++j) tb[g][j] = four(p.B, p.ldb, !BNC, bcol[j], k4);
            }
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                if (kb + (g >> 1) * 16 + 4 * (g & 1) >= p.K) continue;
#pragma unroll
                for (int st = 0; st < 4; ++st)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                ta[g][i][st], tb[g][j][st], acc[i][j], 0, 0, 0);
            }
            if constexpr (kTN)
                if (do_cs)
                    cs.add([&](int k, int c) {
                        const int kk = kb + k;
                        return kk < p.K ? p.B[(size_t)kk * p.ldb + min(n0 + c, p.N - 1)] : 0.0f;
                    });
        }
    }
    __syncthreads();  // every wave past its last tile read before the stage reuse
    if constexpr (kTN)
        if (do_cs) cs.finish(p, lds, n0);
    // The whole tile in bounds: the register epilogue (the choice is uniform
    // across the workgroup, as store_tile has workgroup barriers).
    if (!(p.vec_out && m0 + BM <= p.M && n0 + BN <= p.N &&
          store_direct<TM, TN, IA, IB>(p, acc, m0 + wm0, n0 + wn0, lane)))
        store_tile<TM, TN, WTN, NW, IA, IB>(p, acc, lds, m0 + wm0, n0 + wn0, wave, lane);
}

template <int BM, int BN, int BK, int WGM, int WGN, bool AK, bool BNC, int PRO, bool KT>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_f32_pipe(GemmArgs p) {
    gemm_f32_pipe_body<BM, BN, BK, WGM, WGN, AK, BNC, PRO, KT>(p, blockIdx.x, blockIdx.y);
}

template <int BM, int BN, int WGM, int WGN, int BK, bool AK, bool BNC, int PRO, bool KT = false>
void launch_pipe(const GemmArgs &a0, hipStream_t st) {
    GemmArgs a = a0;
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    const int splits = a.ksplit > 0 ? (a.K + a.ksplit - 1) / a.ksplit : 1;
    gemm_f32_pipe<BM, BN, BK, WGM, WGN, AK, BNC, PRO, KT>
        <<<dim3(a.tiles_m * a.tiles_n, splits), 64 * WGM * WGN, 0, st>>>(a);
}

template <int BM, int BN, int WGM, int WGN, int BK, bool AK, bool BNC, bool VEC, int PRO>
void launch_one(const GemmArgs &a0, hipStream_t st) {
    GemmArgs a = a0;
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    const int splits = a.ksplit > 0 ? (a.K + a.ksplit - 1) / a.ksplit : 1;
    gemm_f32_mfma<BM, BN, BK, WGM, WGN, AK, BNC, VEC, PRO>
        <<<dim3(a.tiles_m * a.tiles_n, splits), 64 * WGM * WGN, 0, st>>>(a);
}

// Tile configurations (index: BM x BN, waves, K depth):
//   0: 256x256, 4 waves, BK 16      1: 256x128, 4 waves, BK 16
//   2: 128x256, 4 waves, BK 16      3: 128x128, 4 waves, BK 32
//   4:  64x64,  4 waves, BK 16      5: 128x64,  4 waves, BK 32
//   6: 256x256, 8 waves, BK 32      7: 256x128, 8 waves, BK 32
// 64x64 is also the only scalar-load variant, for unaligned operands.
constexpr int kNumCfgs = 8;

// K depth of a configuration.
inline int cfg_bk(int cfg) { return (cfg == 3 || cfg >= 5) ? 32 : (cfg == 4 ? 16 : kBK); }

// Output tile of a configuration (the element-load variant is 64x64).
inline void cfg_tile(int cfg, bool vec, int &bm, int &bn) {
    static const int kBm[kNumCfgs] = {256, 256, 128, 128, 64, 128, 256, 256};
    static const int kBn[kNumCfgs] = {256, 128, 256, 128, 64, 64, 256, 128};
    bm = vec ? kBm[cfg] : 64;
    bn = vec ? kBn[cfg] : 64;
}

// Configuration used with a prologue: the 256x256 tiles load directly into
// LDS, which leaves no point to scale a tile at, so they give way to the
// 256x128 tile with the same waves.
inline int pro_cfg(int cfg) { return cfg == 0 ? 1 : cfg == 6 ? 7 : cfg; }

// pipe: the VEC conditions hold (the host checks): the pipelined kernel with
// the same tile shape, over whole K tiles, or (ktail, no prologue) with a
// zero-filled last tile.  With PRO != 0 or ktail the host has mapped cfg
// through pro_cfg (staged tiles).
template <bool AK, bool BNC, int PRO>
void launch_layout(const GemmArgs &a, bool vec, bool pipe, bool ktail, int cfg, hipStream_t st) {
    if (!vec) {
        launch_one<64, 64, 2, 2, 16, AK, BNC, false, PRO>(a, st);
        return;
    }
    if constexpr (PRO == kProNone) {
        if (pipe && ktail) {
            switch (cfg) {
                case 1: launch_pipe<256, 128, 2, 2, kBK, AK, BNC, PRO, true>(a, st); break;
                case 2: launch_pipe<128, 256, 2, 2, kBK, AK, BNC, PRO, true>(a, st); break;
                case 3: launch_pipe<128, 128, 2, 2, 32, AK, BNC, PRO, true>(a, st); break;
                case 5: launch_pipe<128, 64, 2, 2, 32, AK, BNC, PRO, true>(a, st); break;
                case 7: launch_pipe<256, 128, 4, 2, 32, AK, BNC, PRO, true>(a, st); break;
                default: launch_pipe<64, 64, 2, 2, 16, AK, BNC, PRO, true>(a, st); break;
            }
            return;
        }
    }
    if (pipe) {
        switch (cfg) {
            case 0:
                if constexpr (PRO == kProNone) launch_pipe<256, 256, 2, 2, kBK, AK, BNC, PRO>(a, st);
                break;
            case 1: launch_pipe<256, 128, 2, 2, kBK, AK, BNC, PRO>(a, st); break;
            case 2: launch_pipe<128, 256, 2, 2, kBK, AK, BNC, PRO>(a, st); break;
            case 3: launch_pipe<128, 128, 2, 2, 32, AK, BNC, PRO>(a, st); break;
            case 5: launch_pipe<128, 64, 2, 2, 32, AK, BNC, PRO>(a, st); break;
            case 6:
                if constexpr (PRO == kProNone) launch_pipe<256, 256, 2, 4, 32, AK, BNC, PRO>(a, st);
                break;
            case 7: launch_pipe<256, 128, 4, 2, 32, AK, BNC, PRO>(a, st); break;
            default: launch_pipe<64, 64, 2, 2, 16, AK, BNC, PRO>(a, st); break;
        }
        return;
    }
    switch (cfg) {
        case 0:
            if constexpr (PRO == kProNone) launch_one<256, 256, 2, 2, kBK, AK, BNC, true, PRO>(a, st);
            break;
        case 1: launch_one<256, 128, 2, 2, kBK, AK, BNC, true, PRO>(a, st); break;
        case 2: launch_one<128, 256, 2, 2, kBK, AK, BNC, true, PRO>(a, st); break;
        case 3: launch_one<128, 128, 2, 2, 32, AK, BNC, true, PRO>(a, st); break;
        case 5: launch_one<128, 64, 2, 2, 32, AK, BNC, true, PRO>(a, st); break;
        case 6:
            if constexpr (PRO == kProNone) launch_one<256, 256, 2, 4, 32, AK, BNC, true, PRO>(a, st);
            break;
        case 7: launch_one<256, 128, 4, 2, 32, AK, BNC, true, PRO>(a, st); break;
        default: launch_one<64, 64, 2, 2, 16, AK, BNC, true, PRO>(a, st); break;
    }
}

// Defined in k_gemm_{nn,nt,tn}.hip.
// pro: kProNone, or for NT kProAReLU / kProAGelu, for TN kProBReLU / kProBGelu
// (never with ktail).
void launch_nn(const GemmArgs &a, bool vec, bool pipe, bool ktail, int cfg, hipStream_t st);
void launch_nt(const GemmArgs &a, bool vec, bool pipe, bool ktail, int cfg, int pro,
               hipStream_t st);
void launch_tn(const GemmArgs &a, bool vec, bool pipe, bool ktail, int cfg, int pro,
               hipStream_t st);
// The prologue instances (k_gemm_{nt,tn}_pro.hip), pro != kProNone.
void launch_nt_pro(const GemmArgs &a, bool vec, bool pipe, int cfg, int pro, hipStream_t st);
void launch_tn_pro(const GemmArgs &a, bool vec, bool pipe, int cfg, int pro, hipStream_t st);

// Skinny GEMMs (k_gemm_skinny.hip): N <= kSkinnyN and K <= kSkinnyK, any
// layout (0 NN, 1 NT, 2 TN), no prologue, no split; one workgroup per 16
// output rows loads its whole A row panel and the B panel at once.  Takes
// the epilogue (bias, act, Z, act'(Zs), accumulate) and the TN column sums.
constexpr int kSkinnyN = 16;
constexpr int kSkinnyK = 256;
void launch_skinny(const GemmArgs &a, int layout, hipStream_t st);
// NN skinny GEMM whose A operand is the output of the split-K GEMM `pre`
// (its slices written, not yet summed): sums them with pre's epilogue as it
// loads its A panel, and writes pre's outputs; the same bits as the summing
// kernel followed by launch_skinny.  Conditions on the host
// (fg::gemm_fwd_chain_f32): pre splits into at most kSkPreMaxSlices slices,
// its N (a.K) is a multiple of 4 and pre.vec_out holds.
// With `ce` (fg_internal.h) the kernel also finishes the softmax + CE of
// the rows it computes (a head of at most 16 columns).
constexpr int kSkPreMaxSlices = 12;
}  // namespace gemm
struct CeOut;
namespace gemm {
void launch_skinny_pre(const GemmArgs &a, const GemmArgs &pre, hipStream_t st,
                       const CeOut *ce = nullptr);

// A layer's dW (TN, GEMM 1) and dX (NT, GEMM 2) in one launch
// (k_gemm_pair.hip): kinds of the kernels they would take alone.  x1 / x2:
// output tiles (skinny: its workgroups), n1 / n2: workgroups (tiles x K
// slices).  tiles_m / tiles_n of each GemmArgs are set by the caller.
// The first three kinds (256 threads, small LDS) pair with each other; the
// last two only with their own kind, both bodies then sharing one LDS buffer:
// kPairBig: the 8-wave pipelined tiles of large layers, dW on 256x256 (cfg
// 6, TN) with dX on 256x128 (cfg 7, NT), 512 threads;
// kPairMid: both on the 4-wave 128x64 pipelined tiles (cfg 5), 256 threads.
enum : int { kPairSkinny = 0, kPairElem = 1, kPairPipe = 2, kPairBig = 3, kPairMid = 4 };
inline bool pair_exclusive(int kind) { return kind == kPairBig || kind == kPairMid; }
void launch_pair(int k1, int k2, const GemmArgs &a1, const GemmArgs &a2, int x1, int n1, int x2,
                 int n2, hipStream_t st);
// A skinny TN weight gradient (n1 workgroups) with a pair (kinds k2, k3 as
// launch_pair) in one launch.
void launch_triple(const GemmArgs &a1, int n1, int k2, const GemmArgs &a2, int x2, int n2, int k3,
                   const GemmArgs &a3, int x3, int n3, hipStream_t st);

}  // namespace gemm
}  // namespace fg
