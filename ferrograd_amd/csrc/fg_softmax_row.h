// fg_softmax_row.h -- softmax + cross-entropy of a row held in 16 lanes of a
// wave (heads of at most 16 columns): the one-workgroup kernel of
// k_softmax.hip (softmax_ce_tiny) and the skinny head GEMM that finishes a
// captured step's loss itself (fg_gemm_skinny.h) run the same code, so the
// two give the same bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "fg_half.h"

namespace fg {
namespace smrow {

constexpr int kCols = 16;   // columns per row group (lanes)
constexpr int kSlots = 64;  // row slots of the one-workgroup kernel (1024 threads / 16)

// (max, lowest index of the max): the first maximum wins ties.
__device__ __forceinline__ void argmax_combine(float &m, int &i, float m2, int i2) {
    if (m2 > m || (m2 == m && i2 < i)) {
        m = m2;
        i = i2;
    }
}

// DPP controls within a row of 16 lanes: quad permutations [1,0,3,2] and
// [2,3,0,1], the half-row mirror (lane i <-> 7 - i of each 8) and the row
// mirror (lane i <-> 15 - i).
constexpr int kDppSwap1 = 0xB1, kDppSwap2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
template <int CTRL>
__device__ __forceinline__ void row16_step(float &s) {
    s += dpp_f<CTRL>(s);
}
template <int CTRL>
__device__ __forceinline__ void row16_step(float &m, int &am) {
    argmax_combine(m, am, dpp_f<CTRL>(m), dpp_i<CTRL>(am));
}
// Sum / max and first argmax over the 16 lanes of each row group (all lanes
// of the wave active).  Each step combines a lane's value with another's by
// a commutative operation, so every lane of a row ends with the same value,
// the sum always in the same order.
__device__ __forceinline__ float row16_sum(float s) {
    row16_step<kDppSwap1>(s);
    row16_step<kDppSwap2>(s);
    row16_step<kDppHalfMirror>(s);
    row16_step<kDppMirror>(s);
    return s;
}
__device__ __forceinline__ void row16_argmax(float &m, int &am) {
    row16_step<kDppSwap1>(m, am);
    row16_step<kDppSwap2>(m, am);
    row16_step<kDppHalfMirror>(m, am);
    row16_step<kDppMirror>(m, am);
}

template <int DT>
__device__ __forceinline__ void store_as(void *p, uint64_t i, float v) {
    if constexpr (DT == kF32) static_cast<float *>(p)[i] = v;
    else static_cast<uint16_t *>(p)[i] = f_to_h16(DT, v);
}

// Row r (valid: r < R) in lane c of its 16-lane group: v = its logit (lanes
// c >= C hold -inf), t = its label.  Writes argmax, the row loss (lane 0),
// dlogits = scale * (p - [c == t]) (no one-hot without labels) and the
// probabilities, each output optional; returns the row loss (NaN for a
// label outside [0, C)) when want_loss, and in *dl (when given) the lane's
// dlogit as stored (0 for lanes past C or an invalid row).  Called by all 64
// lanes of the wave.
template <int DT>
__device__ __forceinline__ float ce_row16(float v, uint32_t t, int c, int C, int r, bool valid,
                                          bool labels, float scale, float *row_loss, void *out,
                                          int ldo, uint32_t *argmax, void *probs, int ldp,
                                          bool want_loss, float *dl = nullptr) {
    if (dl) *dl = 0.0f;
    float m = v;
    int am = c < C ? c : C;
    row16_argmax(m, am);
    const float e = c < C ? expf(v - m) : 0.0f;
    const float s = row16_sum(e);
    const float xt = row16_sum((c < C && (uint32_t)c == t) ? v : 0.0f);
    if (!valid) return 0.0f;
    if (argmax && c == 0) argmax[r] = (uint32_t)am;
    float l = 0.0f;
    if (want_loss) {
        l = (t < (uint32_t)C) ? (m + logf(s)) - xt : __builtin_nanf("");
        if (row_loss && c == 0) row_loss[r] = l;
    }
    if ((out || probs) && c < C) {
        const float pv = e * (1.0f / s);
        if (out) {
            const float d = scale * (labels && (uint32_t)c == t ? pv - 1.0f : pv);
            store_as<DT>(out, (uint64_t)r * ldo + c, d);
            if (dl) *dl = d;
        }
        if (probs) store_as<DT>(probs, (uint64_t)r * ldp + c, pv);
    }
    return l;
}

// The mean of R row losses in the one-workgroup kernel's order: slot q sums
// rows q, q + kSlots, ... in double, then the slots in order.  One
// workgroup of at least kSlots threads; sh holds kSlots doubles.
__device__ __forceinline__ void mean_rows(const float *row_loss, int R, float *mean, double *sh) {
    if ((int)threadIdx.x < kSlots) {
        double acc = 0.0;
        for (int r = threadIdx.x; r < R; r += kSlots) acc += (double)row_loss[r];
        sh[threadIdx.x] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double tot = sh[0];
        for (int k = 1; k < kSlots; ++k) tot += sh[k];
        mean[0] = (float)(tot / (double)R);
    }
}

}  // namespace smrow
}  // namespace fg
